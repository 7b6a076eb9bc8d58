// C ABI over the C++ API (include/tosa_mi355x.h). Every entry point catches
// all exceptions and turns them into a tosa_status plus a thread-local
// message.
#include <cstring>

#include "../../include/tosa_mi355x.h"
#include "interpreter.h"
#include "kernels.h"
#include "opapi.h"

using namespace tosa;

struct tosa_graph {
    Interpreter interp;
};

struct tosa_tensor {
    TensorPtr t;
};

enum HookKind { HK_CALLBACKS, HK_NOOP, HK_STATS, HK_FLOPS, HK_TRACE, HK_SET };

struct tosa_hook {
    HookKind kind;
    InterpreterHook* impl;                   // owned unless `borrowed`
    bool borrowed = false;
    std::vector<std::unique_ptr<tosa_hook>> members;  // HK_SET: wrappers of the set's hooks
    ~tosa_hook()
    {
        if (!borrowed)
            delete impl;
    }
};

namespace {

thread_local std::string t_last_error;

tosa_status fail(tosa_status s, const std::string& msg)
{
    t_last_error = msg;
    return s;
}

template <typename F>
tosa_status guard(F&& f)
{
    try {
        t_last_error.clear();
        f();
        return TOSA_OK;
    } catch (const Error& e) {
        return fail(static_cast<tosa_status>(e.kind), e.what());
    } catch (const std::bad_alloc&) {
        return fail(TOSA_ERR_DEVICE, "out of host memory");
    } catch (const std::exception& e) {
        return fail(TOSA_ERR_GRAPH, e.what());
    }
}

const BasicBlock* main_block(const tosa_graph* g) { return g ? g->interp.graph().main_block() : nullptr; }

// Temporary handles for callback arguments.
struct Handles {
    std::vector<tosa_tensor> store;
    std::vector<const tosa_tensor*> ptrs;
    explicit Handles(const TensorRefs& refs)
    {
        store.reserve(refs.size());
        for (const Tensor* t : refs) {
            // Non-owning alias: valid for the duration of the callback.
            store.push_back(tosa_tensor{TensorPtr(TensorPtr(), const_cast<Tensor*>(t))});
        }
        for (auto& h : store)
            ptrs.push_back(&h);
    }
};

class CallbackHook : public InterpreterHook {
public:
    explicit CallbackHook(const tosa_hook_callbacks& cb) : cb_(cb) {}
    void pre_op(const OpInfo& o, const TensorRefs& in) override
    {
        if (!cb_.pre_op)
            return;
        Handles h(in);
        cb_.pre_op(cb_.user, o.op, o.op_index, h.ptrs.data(), h.ptrs.size());
    }
    void post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out) override
    {
        if (!cb_.post_op)
            return;
        Handles hi(in), ho(out);
        cb_.post_op(cb_.user, o.op, o.op_index, hi.ptrs.data(), hi.ptrs.size(), ho.ptrs.data(), ho.ptrs.size());
    }
    void on_tensor_alloc(const std::string& n, const Shape& s, DType t, size_t b) override
    {
        if (cb_.on_tensor_alloc)
            cb_.on_tensor_alloc(cb_.user, n.c_str(), s.data(), int(s.size()), uint32_t(t), b);
    }
    void on_tensor_free(const std::string& n, size_t b) override
    {
        if (cb_.on_tensor_free)
            cb_.on_tensor_free(cb_.user, n.c_str(), b);
    }
    bool needs_sync() const override { return cb_.needs_sync != 0; }
    bool reads_data() const override { return cb_.reads_data != 0; }

private:
    tosa_hook_callbacks cb_;
};

tosa_hook* new_hook(HookKind k, InterpreterHook* impl)
{
    auto* h = new tosa_hook();
    h->kind = k;
    h->impl = impl;
    return h;
}

TensorMap input_map(tosa_tensor* const* inputs, size_t n)
{
    TensorMap m;
    for (size_t i = 0; i < n; i++) {
        if (!inputs || !inputs[i] || !inputs[i]->t)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null input tensor");
        m[inputs[i]->t->name] = inputs[i]->t;
    }
    return m;
}

void export_outputs(const TensorMap& out, tosa_tensor*** outputs, size_t* n_outputs)
{
    if (!outputs || !n_outputs)
        throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null output pointer");
    auto** arr = new tosa_tensor*[out.size() ? out.size() : 1];
    size_t i = 0;
    for (const auto& kv : out)
        arr[i++] = new tosa_tensor{kv.second};
    *outputs = arr;
    *n_outputs = out.size();
}

TensorPtr make_named(const char* name, const int64_t* shape, int rank, uint32_t dtype, size_t bytes)
{
    if (rank < 0 || (rank > 0 && !shape))
        throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "bad shape");
    auto t = std::make_shared<Tensor>();
    t->name = name ? name : "";
    t->shape.assign(shape, shape + rank);
    for (int64_t d : t->shape)
        if (d < 0)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "negative dimension");
    const DType dt = static_cast<DType>(dtype);
    if (dtype_size(dt) == 0)
        throw Error(ERR_DTYPE_MISMATCH, std::string("unsupported tensor dtype code ") + std::to_string(dtype));
    const size_t need = size_t(shape_count(t->shape)) * dtype_size(dt);
    if (bytes != need)
        throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT),
                    "expected " + std::to_string(need) + " bytes of element data, got " + std::to_string(bytes));
    return t;
}

}  // namespace

extern "C" {

const char* tosa_last_error(void) { return t_last_error.c_str(); }
const char* tosa_op_name(uint32_t op) { return op_name(op); }
const char* tosa_dtype_name(uint32_t dtype) { return dtype_name(static_cast<DType>(dtype)); }

tosa_status tosa_graph_from_flatbuffer(const uint8_t* data, size_t len, tosa_graph** out)
{
    return guard([&] {
        if (!out)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null output pointer");
        *out = nullptr;
        *out = new tosa_graph{Interpreter::from_flatbuffer(data, len)};
    });
}

void tosa_graph_free(tosa_graph* g) { delete g; }

size_t tosa_graph_num_operators(const tosa_graph* g)
{
    const BasicBlock* b = main_block(g);
    return b ? b->operators.size() : 0;
}

tosa_status tosa_graph_operator(const tosa_graph* g, size_t i, uint32_t* op, size_t* n_inputs, size_t* n_outputs)
{
    const BasicBlock* b = main_block(g);
    if (!b || i >= b->operators.size())
        return fail(TOSA_ERR_INVALID_ARGUMENT, "operator index out of range");
    const Operator& o = b->operators[i];
    if (op)
        *op = o.op;
    if (n_inputs)
        *n_inputs = o.inputs.size();
    if (n_outputs)
        *n_outputs = o.outputs.size();
    return TOSA_OK;
}

const char* tosa_graph_operator_input(const tosa_graph* g, size_t i, size_t j)
{
    const BasicBlock* b = main_block(g);
    if (!b || i >= b->operators.size() || j >= b->operators[i].inputs.size())
        return nullptr;
    return b->operators[i].inputs[j].c_str();
}

const char* tosa_graph_operator_output(const tosa_graph* g, size_t i, size_t j)
{
    const BasicBlock* b = main_block(g);
    if (!b || i >= b->operators.size() || j >= b->operators[i].outputs.size())
        return nullptr;
    return b->operators[i].outputs[j].c_str();
}

size_t tosa_graph_num_tensors(const tosa_graph* g)
{
    const BasicBlock* b = main_block(g);
    return b ? b->tensors.size() : 0;
}

tosa_status tosa_graph_tensor(const tosa_graph* g, size_t i, const char** name, uint32_t* dtype, int32_t* shape,
                              int cap, int* rank, int* has_data)
{
    const BasicBlock* b = main_block(g);
    if (!b || i >= b->tensors.size())
        return fail(TOSA_ERR_INVALID_ARGUMENT, "tensor index out of range");
    const TensorDef& t = b->tensors[i];
    if (name)
        *name = t.name.c_str();
    if (dtype)
        *dtype = uint32_t(t.dtype);
    if (rank)
        *rank = int(t.shape.size());
    if (has_data)
        *has_data = t.has_data ? 1 : 0;
    if (shape)
        for (int k = 0; k < cap && k < int(t.shape.size()); k++)
            shape[k] = t.shape[k];
    return TOSA_OK;
}

size_t tosa_graph_num_inputs(const tosa_graph* g)
{
    const BasicBlock* b = main_block(g);
    return b ? b->inputs.size() : 0;
}
size_t tosa_graph_num_outputs(const tosa_graph* g)
{
    const BasicBlock* b = main_block(g);
    return b ? b->outputs.size() : 0;
}
const char* tosa_graph_input(const tosa_graph* g, size_t i)
{
    const BasicBlock* b = main_block(g);
    return (b && i < b->inputs.size()) ? b->inputs[i].c_str() : nullptr;
}
const char* tosa_graph_output(const tosa_graph* g, size_t i)
{
    const BasicBlock* b = main_block(g);
    return (b && i < b->outputs.size()) ? b->outputs[i].c_str() : nullptr;
}

tosa_status tosa_tensor_from_host(const char* name, const int64_t* shape, int rank, uint32_t dtype, const void* data,
                                  size_t bytes, tosa_tensor** out)
{
    return guard([&] {
        if (!out || (bytes && !data))
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null pointer");
        TensorPtr t = make_named(name, shape, rank, dtype, bytes);
        t->data = make_host_storage(static_cast<DType>(dtype), shape_count(t->shape), data);
        *out = new tosa_tensor{t};
    });
}

tosa_status tosa_tensor_from_device(const char* name, const int64_t* shape, int rank, uint32_t dtype, void* dev_ptr,
                                    size_t bytes, tosa_tensor** out)
{
    return guard([&] {
        if (!out || (bytes && !dev_ptr))
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null pointer");
        TensorPtr t = make_named(name, shape, rank, dtype, bytes);
        t->data = wrap_device_storage(static_cast<DType>(dtype), shape_count(t->shape), dev_ptr);
        *out = new tosa_tensor{t};
    });
}

tosa_status tosa_tensor_to_host(const tosa_tensor* t, void* dst, size_t bytes)
{
    return guard([&] {
        if (!t || !t->t || !t->t->data)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null tensor");
        const size_t have = t->t->data->bytes();
        if (bytes != have)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT),
                        "tensor holds " + std::to_string(have) + " bytes, buffer has " + std::to_string(bytes));
        if (have && !dst)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null destination");
        const uint8_t* p = t->t->data->host_in();
        if (have)
            std::memcpy(dst, p, have);
    });
}

tosa_status tosa_tensor_device_ptr(const tosa_tensor* t, const void** ptr)
{
    return guard([&] {
        if (!t || !t->t || !t->t->data || !ptr)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null pointer");
        *ptr = t->t->data->device_in();
    });
}

const char* tosa_tensor_name(const tosa_tensor* t) { return (t && t->t) ? t->t->name.c_str() : nullptr; }
uint32_t tosa_tensor_dtype(const tosa_tensor* t) { return (t && t->t) ? uint32_t(t->t->dtype()) : 0u; }
int tosa_tensor_rank(const tosa_tensor* t) { return (t && t->t) ? int(t->t->shape.size()) : -1; }

tosa_status tosa_tensor_shape(const tosa_tensor* t, int64_t* dims, int cap)
{
    if (!t || !t->t)
        return fail(TOSA_ERR_INVALID_ARGUMENT, "null tensor");
    for (int k = 0; k < cap && k < int(t->t->shape.size()); k++)
        dims[k] = t->t->shape[k];
    return TOSA_OK;
}

size_t tosa_tensor_size_bytes(const tosa_tensor* t) { return (t && t->t) ? t->t->size_bytes() : 0; }
size_t tosa_tensor_data_bytes(const tosa_tensor* t) { return (t && t->t && t->t->data) ? t->t->data->bytes() : 0; }
void tosa_tensor_free(tosa_tensor* t) { delete t; }

tosa_hook* tosa_hook_new_callbacks(const tosa_hook_callbacks* cb)
{
    if (!cb)
        return nullptr;
    return new_hook(HK_CALLBACKS, new CallbackHook(*cb));
}
tosa_hook* tosa_hook_new_noop(void) { return new_hook(HK_NOOP, new NoopHook()); }
tosa_hook* tosa_hook_new_stats(void) { return new_hook(HK_STATS, new StatsCollector()); }
tosa_hook* tosa_hook_new_flops(void) { return new_hook(HK_FLOPS, new FlopCounter()); }
tosa_hook* tosa_hook_new_trace(void) { return new_hook(HK_TRACE, new OpTrace()); }
tosa_hook* tosa_hook_new_set(void) { return new_hook(HK_SET, new HookSet()); }

tosa_status tosa_hookset_add(tosa_hook* set, tosa_hook* hook)
{
    if (!set || set->kind != HK_SET || !hook || hook->borrowed)
        return fail(TOSA_ERR_INVALID_ARGUMENT, "tosa_hookset_add needs a hook set and an owned hook");
    auto* hs = static_cast<HookSet*>(set->impl);
    hs->add(std::unique_ptr<InterpreterHook>(hook->impl));
    hook->borrowed = true;  // the set owns the implementation now
    set->members.emplace_back(hook);
    return TOSA_OK;
}

size_t tosa_hookset_len(const tosa_hook* set)
{
    return (set && set->kind == HK_SET) ? set->members.size() : 0;
}

tosa_hook* tosa_hookset_get(tosa_hook* set, size_t i)
{
    if (!set || set->kind != HK_SET || i >= set->members.size())
        return nullptr;
    return set->members[i].get();
}

void tosa_hook_free(tosa_hook* h)
{
    if (h && h->borrowed)
        return;  // owned by a hook set
    delete h;
}

static const StatsCollector* stats_of(const tosa_hook* h)
{
    return (h && h->kind == HK_STATS) ? static_cast<const StatsCollector*>(h->impl) : nullptr;
}
uint64_t tosa_stats_total_ops(const tosa_hook* h)
{
    auto* s = stats_of(h);
    return s ? s->total_ops_executed : 0;
}
size_t tosa_stats_peak_memory(const tosa_hook* h)
{
    auto* s = stats_of(h);
    return s ? s->peak_memory_bytes : 0;
}
size_t tosa_stats_current_memory(const tosa_hook* h)
{
    auto* s = stats_of(h);
    return s ? s->current_memory_bytes : 0;
}
size_t tosa_stats_num_ops(const tosa_hook* h)
{
    auto* s = stats_of(h);
    return s ? s->op_stats.size() : 0;
}
tosa_status tosa_stats_op(const tosa_hook* h, size_t i, const char** name, uint64_t* count, double* seconds,
                          uint64_t* elements_in, uint64_t* elements_out)
{
    auto* s = stats_of(h);
    if (!s || i >= s->op_stats.size())
        return fail(TOSA_ERR_INVALID_ARGUMENT, "not a stats hook or index out of range");
    auto it = s->op_stats.begin();
    std::advance(it, i);
    if (name)
        *name = it->first.c_str();
    if (count)
        *count = it->second.count;
    if (seconds)
        *seconds = it->second.total_time;
    if (elements_in)
        *elements_in = it->second.total_input_elements;
    if (elements_out)
        *elements_out = it->second.total_output_elements;
    return TOSA_OK;
}
size_t tosa_stats_summary(const tosa_hook* h, char* buf, size_t cap)
{
    auto* s = stats_of(h);
    if (!s)
        return 0;
    const std::string text = s->summary();
    if (buf && cap) {
        const size_t n = std::min(cap - 1, text.size());
        std::memcpy(buf, text.data(), n);
        buf[n] = 0;
    }
    return text.size();
}

static const FlopCounter* flops_of(const tosa_hook* h)
{
    return (h && h->kind == HK_FLOPS) ? static_cast<const FlopCounter*>(h->impl) : nullptr;
}
uint64_t tosa_flops_total(const tosa_hook* h)
{
    auto* f = flops_of(h);
    return f ? f->total_flops : 0;
}
uint64_t tosa_flops_for(const tosa_hook* h, const char* op)
{
    auto* f = flops_of(h);
    if (!f || !op)
        return 0;
    auto it = f->flops_by_op.find(op);
    return it == f->flops_by_op.end() ? 0 : it->second;
}

static const OpTrace* trace_of(const tosa_hook* h)
{
    return (h && h->kind == HK_TRACE) ? static_cast<const OpTrace*>(h->impl) : nullptr;
}
size_t tosa_trace_len(const tosa_hook* h)
{
    auto* t = trace_of(h);
    return t ? t->entries.size() : 0;
}
tosa_status tosa_trace_entry(const tosa_hook* h, size_t i, const char** op, size_t* op_index, size_t* n_inputs,
                             size_t* n_outputs)
{
    auto* t = trace_of(h);
    if (!t || i >= t->entries.size())
        return fail(TOSA_ERR_INVALID_ARGUMENT, "not a trace hook or index out of range");
    const TraceEntry& e = t->entries[i];
    if (op)
        *op = e.op.c_str();
    if (op_index)
        *op_index = e.op_index;
    if (n_inputs)
        *n_inputs = e.input_shapes.size();
    if (n_outputs)
        *n_outputs = e.output_shapes.size();
    return TOSA_OK;
}
tosa_status tosa_trace_shape(const tosa_hook* h, size_t i, int output, size_t j, int64_t* dims, int cap, int* rank)
{
    auto* t = trace_of(h);
    if (!t || i >= t->entries.size())
        return fail(TOSA_ERR_INVALID_ARGUMENT, "not a trace hook or index out of range");
    const auto& v = output ? t->entries[i].output_shapes : t->entries[i].input_shapes;
    if (j >= v.size())
        return fail(TOSA_ERR_INVALID_ARGUMENT, "shape index out of range");
    if (rank)
        *rank = int(v[j].size());
    for (int k = 0; dims && k < cap && k < int(v[j].size()); k++)
        dims[k] = v[j][k];
    return TOSA_OK;
}

tosa_status tosa_run(const tosa_graph* g, tosa_tensor* const* inputs, size_t n_inputs, tosa_hook* hook,
                     tosa_tensor*** outputs, size_t* n_outputs)
{
    return guard([&] {
        if (!g)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null graph");
        NoopHook noop;
        InterpreterHook& h = hook ? *hook->impl : static_cast<InterpreterHook&>(noop);
        TensorMap out = g->interp.run(input_map(inputs, n_inputs), h);
        export_outputs(out, outputs, n_outputs);
    });
}

void tosa_outputs_free(tosa_tensor** outputs, size_t n)
{
    if (!outputs)
        return;
    for (size_t i = 0; i < n; i++)
        delete outputs[i];
    delete[] outputs;
}

void tosa_outputs_array_free(tosa_tensor** outputs) { delete[] outputs; }

tosa_status tosa_run_graph(const uint8_t* data, size_t len, tosa_tensor* const* inputs, size_t n_inputs,
                           tosa_tensor*** outputs, size_t* n_outputs)
{
    return guard([&] { export_outputs(run_graph(data, len, input_map(inputs, n_inputs)), outputs, n_outputs); });
}

tosa_status tosa_run_graph_with_stats(const uint8_t* data, size_t len, tosa_tensor* const* inputs, size_t n_inputs,
                                      tosa_tensor*** outputs, size_t* n_outputs, tosa_hook** stats)
{
    return guard([&] {
        if (!stats)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null stats pointer");
        *stats = nullptr;
        std::unique_ptr<tosa_hook> h(tosa_hook_new_stats());
        TensorMap out =
            run_graph_with_stats(data, len, input_map(inputs, n_inputs), *static_cast<StatsCollector*>(h->impl));
        export_outputs(out, outputs, n_outputs);
        *stats = h.release();
    });
}

tosa_status tosa_run_graph_with_hooks(const uint8_t* data, size_t len, tosa_tensor* const* inputs, size_t n_inputs,
                                      tosa_hook* hooks, tosa_tensor*** outputs, size_t* n_outputs)
{
    return guard([&] {
        if (!hooks)
            throw Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), "null hook");
        export_outputs(run_graph_with_hooks(data, len, input_map(inputs, n_inputs), *hooks->impl), outputs,
                       n_outputs);
    });
}

tosa_status tosa_set_option(const char* key, int value)
{
    if (!key)
        return fail(TOSA_ERR_INVALID_ARGUMENT, "null key");
    RunOptions& o = default_run_options();
    if (std::strcmp(key, "fusion") == 0)
        o.fusion = value != 0;
    else if (std::strcmp(key, "strict_float") == 0)
        o.strict_float = value != 0;
    else if (std::strcmp(key, "deferred") == 0)
        o.deferred = value != 0;
    else if (std::strcmp(key, "conv_rows") == 0)
        kern::set_conv_rows_mode(value);
    else if (std::strcmp(key, "matmul_rows") == 0)
        kern::set_mm_tile_rows(value);
    else
        return fail(TOSA_ERR_INVALID_ARGUMENT, std::string("unknown option ") + key);
    return TOSA_OK;
}

int tosa_get_option(const char* key)
{
    if (!key)
        return -1;
    const RunOptions& o = default_run_options();
    if (std::strcmp(key, "fusion") == 0)
        return o.fusion;
    if (std::strcmp(key, "strict_float") == 0)
        return o.strict_float;
    if (std::strcmp(key, "deferred") == 0)
        return o.deferred;
    if (std::strcmp(key, "conv_rows") == 0)
        return kern::conv_rows_mode();
    if (std::strcmp(key, "matmul_rows") == 0)
        return kern::mm_tile_rows();
    return -1;
}

tosa_status tosa_set_stream(void* hip_stream)
{
    set_thread_stream(static_cast<hipStream_t>(hip_stream));
    return TOSA_OK;
}

tosa_status tosa_synchronize(void)
{
    return guard([] {
        Stream& s = thread_stream();
        const uint32_t e = read_error_word(s);  // synchronises the stream
        if (e) {
            clear_error_word(s);
            throw Error(ERR_GRAPH, device_error_message(e));
        }
    });
}

int tosa_device_count(void) { return device_count(); }

tosa_status tosa_conv2d_i8(const int8_t* x, const int64_t x_shape[4], const int8_t* w, const int64_t w_shape[4],
                           const int32_t* bias, int64_t bias_len, int32_t input_zp, int32_t weight_zp,
                           const int32_t pad[4], const int32_t stride[2], const int32_t dilation[2],
                           const tosa_rescale_i32* rescale, void* out, int64_t out_shape[4],
                           uint32_t* device_error, void* stream)
{
    return guard([&] {
        ConvI8Args a;
        a.x = x;
        a.x_shape = x_shape;
        a.w = w;
        a.w_shape = w_shape;
        a.bias = bias;
        a.bias_len = bias_len;
        a.input_zp = input_zp;
        a.weight_zp = weight_zp;
        a.pad = pad;
        a.stride = stride;
        a.dilation = dilation;
        a.rescale = rescale;
        a.out = out;
        a.device_error = device_error;
        a.stream = stream;
        conv2d_i8(a, out_shape);
    });
}

tosa_status tosa_matmul_i8(const int8_t* a, const int64_t a_shape[3], const int8_t* b, const int64_t b_shape[3],
                           int32_t a_zp, int32_t b_zp, const tosa_rescale_i32* rescale, void* out,
                           int64_t out_shape[3], uint32_t* device_error, void* stream)
{
    return guard([&] {
        MatmulI8OpArgs m;
        m.a = a;
        m.a_shape = a_shape;
        m.b = b;
        m.b_shape = b_shape;
        m.a_zp = a_zp;
        m.b_zp = b_zp;
        m.rescale = rescale;
        m.out = out;
        m.device_error = device_error;
        m.stream = stream;
        matmul_i8(m, out_shape);
    });
}

tosa_status tosa_conv2d_i8_noalloc(const int8_t* x, const int64_t x_shape[4], const int8_t* w,
                                   const int64_t w_shape[4], const int32_t* bias, int64_t bias_len, int32_t input_zp,
                                   int32_t weight_zp, const int32_t pad[4], const int32_t stride[2],
                                   const int32_t dilation[2], const tosa_rescale_i32* rescale, void* out,
                                   int64_t out_shape[4], uint32_t* device_error, void* stream)
{
    return guard([&] {
        ConvI8Args a;
        a.x = x;
        a.x_shape = x_shape;
        a.w = w;
        a.w_shape = w_shape;
        a.bias = bias;
        a.bias_len = bias_len;
        a.input_zp = input_zp;
        a.weight_zp = weight_zp;
        a.pad = pad;
        a.stride = stride;
        a.dilation = dilation;
        a.rescale = rescale;
        a.out = out;
        a.device_error = device_error;
        a.stream = stream;
        conv2d_i8_noalloc(a, out_shape);
    });
}

}  // extern "C"
