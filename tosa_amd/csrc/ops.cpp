// Operator evaluation on the MI355X path: the reference's per-operator
// validation (same checks, same order, same error kinds) followed by a
// kernel launch instead of a host loop. Dispatch mirrors src/ops/mod.rs:22-150
// for the operators of this path; every other operator is rejected as
// unsupported.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <optional>

#include "exec.h"

namespace tosa {

using namespace kern;

// ---------------------------------------------------------------------------
// ExecState / ConstCache
// ---------------------------------------------------------------------------
TensorPtr ExecState::get(const std::string& name) const
{
    auto it = tensors.find(name);
    if (it == tensors.end())
        throw Error(ERR_TENSOR_NOT_FOUND, name);
    return it->second;
}

const TensorDef* ExecState::find_def(const std::string& name) const
{
    auto it = defs->find(name);
    return it == defs->end() ? nullptr : it->second;
}

static Shape shape_from_ir(const std::vector<int32_t>& s)
{
    Shape r;
    r.reserve(s.size());
    for (int32_t d : s)
        r.push_back(d < 0 ? 0 : d);
    return r;
}

StoragePtr ConstCache::get(const TensorDef& def)
{
    std::lock_guard<std::mutex> lk(mu_);
    auto it = map_.find(&def);
    if (it != map_.end())
        return it->second;
    const int64_t count = shape_count(shape_from_ir(def.shape));
    StoragePtr s = def.has_data ? storage_from_raw_bytes(def.dtype, def.data.data(), def.data.size(), count)
                                : storage_zeros(def.dtype, count);
    s->shared_const = true;
    map_[&def] = s;
    return s;
}

TensorPtr ExecState::resolve(const std::string& name) const
{
    auto it = tensors.find(name);
    if (it != tensors.end())
        return it->second;
    auto c = const_defs->find(name);
    if (c == const_defs->end())
        return nullptr;
    try {
        auto t = std::make_shared<Tensor>();
        t->name = name;
        t->shape = shape_from_ir(c->second->shape);
        t->data = consts->get(*c->second);
        return t;
    } catch (const Error&) {
        return nullptr;
    }
}

namespace {

TensorPtr make_tensor(const std::string& name, const Shape& shape, StoragePtr data)
{
    auto t = std::make_shared<Tensor>();
    t->name = name;
    t->shape = shape;
    t->data = std::move(data);
    return t;
}

TensorPtr new_output(const std::string& name, const Shape& shape, DType t)
{
    return make_tensor(name, shape, make_device_storage(t, shape_count(shape)));
}

// A tensor whose storage is computed on demand by `fill` (see Storage).
TensorPtr virtual_output(const std::string& name, const Shape& shape, DType t, std::function<void(Storage&)> fill)
{
    auto s = std::make_shared<Storage>();
    s->dtype = t;
    s->count = shape_count(shape);
    s->materialize = std::move(fill);
    return make_tensor(name, shape, s);
}

// ---------------------------------------------------------------------------
// Shared validation, src/ops/common.rs
// ---------------------------------------------------------------------------
void expect_operands(const Operator& op, const std::string& name, size_t in, size_t out)
{
    if (op.inputs.size() != in || op.outputs.size() != out)
        throw invalid(name, "expected " + std::to_string(in) + " inputs and " + std::to_string(out) +
                                " outputs, got " + std::to_string(op.inputs.size()) + " and " +
                                std::to_string(op.outputs.size()));
}

void expect_rank(const std::string& op, const std::string& what, const Tensor& t, size_t rank)
{
    if (t.shape.size() != rank)
        throw Error(ERR_SHAPE_MISMATCH,
                    op + ": " + what + " must have rank " + std::to_string(rank) + ", got shape " + shape_str(t.shape));
}

TensorPtr single_value(const std::string& op, const std::string& what, TensorPtr t)
{
    expect_rank(op, what, *t, 1);
    if (t->len() != 1)
        throw Error(ERR_SHAPE_MISMATCH,
                    op + ": " + what + " must have exactly one element, got shape " + shape_str(t->shape));
    return t;
}

std::optional<DType> check_declared_output(const ExecState& st, const std::string& op, const std::string& name,
                                           const Shape& shape)
{
    const TensorDef* def = st.find_def(name);
    if (!def)
        return std::nullopt;
    const bool static_shape = std::all_of(def->shape.begin(), def->shape.end(), [](int32_t d) { return d >= 0; });
    if (static_shape) {
        Shape declared(def->shape.begin(), def->shape.end());
        if (declared != shape)
            throw Error(ERR_SHAPE_MISMATCH, op + ": output shape " + shape_str(shape) + " does not match declared shape " +
                                                shape_str(declared));
    }
    return def->dtype;
}

// finish() of the element-wise and data-layout operators: declared shape and
// dtype must match the result.
void check_finish(const ExecState& st, const std::string& op, const std::string& out, const Shape& shape, DType t)
{
    auto d = check_declared_output(st, op, out, shape);
    if (d && *d != t)
        throw Error(ERR_DTYPE_MISMATCH,
                    op + ": output dtype " + dtype_name(*d) + " should be " + dtype_name(t));
}

bool is_fp8(DType t) { return t == DT_FP8E4M3 || t == DT_FP8E5M2; }

ElemCode elem_code(DType t)
{
    switch (t) {
    case DT_BOOL: return E_U8;
    case DT_INT4:
    case DT_INT8: return E_I8;
    case DT_INT16: return E_I16;
    case DT_INT32: return E_I32;
    case DT_INT48:
    case DT_INT64:
    case DT_SHAPE: return E_I64;
    case DT_FP32: return E_F32;
    case DT_FP16: return E_F16;
    case DT_BF16: return E_BF16;
    case DT_FP8E4M3: return E_FP8E4M3;
    case DT_FP8E5M2: return E_FP8E5M2;
    default: throw Error(ERR_DTYPE_MISMATCH, std::string("no device representation for ") + dtype_name(t));
    }
}

int32_t fmt_code(DType t)
{
    switch (t) {
    case DT_FP16: return FMT_F16;
    case DT_BF16: return FMT_BF16;
    case DT_FP8E4M3: return FMT_FP8E4M3;
    case DT_FP8E5M2: return FMT_FP8E5M2;
    default: return FMT_F32;
    }
}

std::pair<int64_t, int64_t> int_range(DType t)
{
    switch (t) {
    case DT_INT4: return {-8, 7};
    case DT_INT8: return {-128, 127};
    case DT_INT16: return {-32768, 32767};
    case DT_INT32: return {INT32_MIN, INT32_MAX};
    case DT_INT48: return {-(int64_t(1) << 47), (int64_t(1) << 47) - 1};
    default: return {INT64_MIN, INT64_MAX};
    }
}

std::mutex& derived_mu()
{
    static std::mutex mu;
    return mu;
}

// Data derived from a graph constant's storage by `make`, built once and
// kept with it. Runs on several threads may share the constant: the slot is
// read and filled under a lock (`make` runs outside it).
StoragePtr cached_aux(Storage& owner, int kind, const std::function<StoragePtr()>& make)
{
    {
        std::lock_guard<std::mutex> lk(derived_mu());
        if (owner.aux && owner.aux_kind == kind)
            return owner.aux;
    }
    StoragePtr made = make();
    std::lock_guard<std::mutex> lk(derived_mu());
    if (!(owner.aux && owner.aux_kind == kind)) {
        owner.aux = made;
        owner.aux_kind = kind;
    }
    return owner.aux;
}

enum AuxKind { AUX_WSUM = 1, AUX_F32 = 2 };

// Epilogue table of the fast int8 convolution for `rs` (the plain int32
// epilogue when null). Cached on the weight storage when everything it is
// built from is a graph constant (`cacheable`); the table kernel then
// completes before the table is shared, so runs on other streams see it.
StoragePtr conv_i8_table_for(const ConvI8Desc& d, Storage& wstore, const void* bias_key, const RescaleDev* rs,
                             bool cacheable, hipStream_t s)
{
    std::string key;
    if (cacheable) {
        char buf[192];
        std::snprintf(buf, sizeof buf, "conv_i8_tab:%d:%d:%p:%d:%d:%d:%p:%p:%d:%d:%lld", d.w != nullptr, d.batch, bias_key,
                      d.bias_len, d.zp_x, d.zp_w, rs ? static_cast<const void*>(rs->mult) : nullptr,
                      rs ? static_cast<const void*>(rs->shift) : nullptr, rs ? rs->per_channel : 0,
                      rs ? rs->rounding : 0, rs ? static_cast<long long>(rs->out_zp) : 0LL);
        key = buf;
        std::lock_guard<std::mutex> lk(derived_mu());
        auto it = wstore.derived.find(key);
        if (it != wstore.derived.end())
            return it->second;
    }
    auto t = make_device_storage(DT_INT32, conv_i8_table_words(d.oc, d.batch));
    conv_i8_table(d, rs, t->device_out(), s);
    if (cacheable) {
        hip_check(hipStreamSynchronize(s), "conv_i8 table");
        // A cached table is read back once: when it rules out every range
        // failure, the kernels drop the per-value check.
        if (rs && rs->min_shift <= 31)
            t->scale_range_safe = conv_i8_table_range_safe(d, t->device_in());
        std::lock_guard<std::mutex> lk(derived_mu());
        wstore.derived[key] = t;
    }
    return t;
}

// Packed weights of the stride-1 halo convolution kernel (null when it does
// not run for `d`), cached on the weight storage when the weight is a graph
// constant.
StoragePtr conv_i8_wpack_for(const ConvI8Desc& d, Storage& wstore, bool cacheable, hipStream_t s)
{
    const int64_t bytes = conv_i8_wpack_bytes(d);
    if (bytes <= 0)
        return nullptr;
    const std::string key = "conv_i8_wpack:" + std::to_string(bytes) + ":" + std::to_string(conv_i8_wpack_block(d));
    if (cacheable) {
        std::lock_guard<std::mutex> lk(derived_mu());
        auto it = wstore.derived.find(key);
        if (it != wstore.derived.end())
            return it->second;
    }
    auto t = make_device_storage(DT_INT8, bytes);
    conv_i8_wpack(d, t->device_out(), s);
    if (cacheable) {
        hip_check(hipStreamSynchronize(s), "conv_i8 weight pack");
        std::lock_guard<std::mutex> lk(derived_mu());
        wstore.derived[key] = t;
    }
    return t;
}

// Device data derived from a weight-like operand by `make` (an int8 buffer
// of `bytes`), cached on its storage under `key` when the operand is a graph
// constant.
StoragePtr derived_i8(Storage& wstore, const std::string& key, int64_t bytes, bool cacheable, hipStream_t s,
                      const std::function<void(void*)>& make)
{
    if (cacheable) {
        std::lock_guard<std::mutex> lk(derived_mu());
        auto it = wstore.derived.find(key);
        if (it != wstore.derived.end())
            return it->second;
    }
    auto t = make_device_storage(DT_INT8, bytes);
    make(t->device_out());
    if (cacheable) {
        hip_check(hipStreamSynchronize(s), key.c_str());
        std::lock_guard<std::mutex> lk(derived_mu());
        wstore.derived[key] = t;
    }
    return t;
}

// ---------------------------------------------------------------------------
// RESCALE preparation: every check of eval_rescale (src/ops/type_conv.rs:
// 111-170) plus the host-side parameter check that apply_scale_32/16 would
// fail on (multiplier < 0, shift outside [2, 62]).
// ---------------------------------------------------------------------------
int bit_width(DType t) { return t == DT_INT8 ? 8 : t == DT_INT16 ? 16 : t == DT_INT32 ? 32 : 48; }

struct RescalePrep {
    DType in_t, out_t;
    Shape shape;
    RescaleDev rs;
    StoragePtr params;  // [mult(channels) | shift(channels)] int32 on device
};

RescalePrep prepare_rescale(const ExecState& st, const Operator& op, const Tensor& input, TensorPtr multiplier,
                            TensorPtr shift, TensorPtr in_zp, TensorPtr out_zp)
{
    const std::string OP = "RESCALE";
    const OpAttribute& a = op.attr;
    RescalePrep p;
    p.shape = input.shape;
    p.in_t = input.dtype();
    p.out_t = check_declared_output(st, OP, op.outputs[0], p.shape).value_or(DT_INT32);
    const DType in_t = p.in_t, out_t = p.out_t;
    const bool in_ok = in_t == DT_INT8 || in_t == DT_INT16 || in_t == DT_INT32 || in_t == DT_INT48;
    const bool out_ok = out_t == DT_INT8 || out_t == DT_INT16 || out_t == DT_INT32;
    if (!in_ok || !out_ok)
        throw Error(ERR_DTYPE_MISMATCH,
                    OP + ": unsupported types " + dtype_name(in_t) + " -> " + dtype_name(out_t));
    if (a.rounding_mode == ROUND_UNKNOWN)
        throw invalid(OP, "unsupported rounding mode");
    if (a.scale32 && in_t == DT_INT48)
        throw invalid(OP, "scale32 is not allowed for INT48 input");
    if (!a.scale32 && a.rounding_mode == ROUND_DOUBLE)
        throw invalid(OP, "double rounding requires scale32");
    const bool has32 = in_t == DT_INT32 || in_t == DT_INT48 || out_t == DT_INT32;
    if ((a.input_unsigned && a.output_unsigned) || ((a.input_unsigned || a.output_unsigned) && has32))
        throw invalid(OP, "invalid combination of input_unsigned/output_unsigned and types");
    const DType want_m = a.scale32 ? DT_INT32 : DT_INT16;
    if (multiplier->dtype() != want_m || shift->dtype() != DT_INT8)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": multiplier must be " + dtype_name(want_m) + " and shift INT8, got " +
                                            dtype_name(multiplier->dtype()) + "/" + dtype_name(shift->dtype()));
    if (in_zp->dtype() != in_t || out_zp->dtype() != out_t || in_zp->len() != 1 || out_zp->len() != 1)
        throw invalid(OP, "zero points must be single elements of the input/output types");
    int64_t channels = 1;
    if (a.per_channel) {
        if (p.shape.empty())
            throw invalid(OP, "per_channel requires rank >= 1");
        channels = p.shape.back();
    }
    if (multiplier->len() != channels || shift->len() != channels)
        throw invalid(OP, "multiplier and shift must have " + std::to_string(channels) + " elements");
    auto extend = [](DType t, int64_t v, bool u) { return u ? (v & ((int64_t(1) << bit_width(t)) - 1)) : v; };
    const int64_t izp = extend(in_t, int_values(*in_zp)[0], a.input_unsigned);
    const int64_t ozp = extend(out_t, int_values(*out_zp)[0], a.output_unsigned);
    auto zp_ok = [](DType t, int64_t zp, bool u) { return t == DT_INT8 || zp == 0 || (t == DT_INT16 && u && zp == 32768); };
    if (!zp_ok(in_t, izp, a.input_unsigned) || !zp_ok(out_t, ozp, a.output_unsigned))
        throw invalid(OP, "zero point not allowed for this type");

    // Multiplier and shift as int32 on the device. For graph constants they
    // are built once per (multiplier, shift) pair and kept with the
    // multiplier (never replaced, so their device address identifies them
    // for as long as the graph lives); other operands are re-read and
    // uploaded on every run, since their memory may change between runs.
    const bool params_const = st.is_const(op.inputs[1]) && st.is_const(op.inputs[2]);
    Storage& ms = *multiplier->data;
    char key[64];
    std::snprintf(key, sizeof key, "rescale_params:%p", static_cast<const void*>(shift->data.get()));
    if (params_const) {
        std::lock_guard<std::mutex> lk(derived_mu());
        auto it = ms.derived.find(key);
        if (it != ms.derived.end())
            p.params = it->second;
    }
    std::vector<int64_t> mv = int_values(*multiplier), sv = int_values(*shift);
    if (shape_count(p.shape) > 0 && a.rounding_mode != ROUND_INEXACT) {
        for (int64_t c = 0; c < channels; c++) {
            const int64_t m = a.scale32 ? int64_t(int32_t(mv[c])) : int64_t(int16_t(mv[c]));
            const int64_t s = int32_t(sv[c]);
            if (m < 0 || s < 2 || s > 62)
                throw Error(ERR_GRAPH, std::string(a.scale32 ? "apply_scale_32" : "apply_scale_16") +
                                           ": invalid multiplier " + std::to_string(m) + " or shift " +
                                           std::to_string(s));
        }
    }
    if (!p.params) {
        std::vector<int32_t> host(2 * channels);
        for (int64_t c = 0; c < channels; c++) {
            host[c] = int32_t(mv[c]);
            host[channels + c] = int32_t(sv[c]);
        }
        p.params = make_host_storage(DT_INT32, 2 * channels, host.data());
        if (params_const) {
            p.params->shared_const = true;
            std::lock_guard<std::mutex> lk(derived_mu());
            auto ins = ms.derived.emplace(key, p.params);
            p.params = ins.first->second;  // another run may have built it first
        }
    }
    const int32_t* dp = static_cast<const int32_t*>(p.params->device_in());
    RescaleDev& r = p.rs;
    r.mult = dp;
    r.shift = dp + channels;
    r.channels = int32_t(channels);
    r.per_channel = a.per_channel;
    r.scale32 = a.scale32;
    r.rounding = int32_t(a.rounding_mode);
    r.in_bits = bit_width(in_t);
    r.in_unsigned = a.input_unsigned;
    r.in_zp = izp;
    r.out_zp = ozp;
    r.max_shift = 2;
    r.min_shift = 62;
    for (int64_t c = 0; c < channels; c++) {
        r.max_shift = std::max<int32_t>(r.max_shift, int32_t(sv[c]));
        r.min_shift = std::min<int32_t>(r.min_shift, int32_t(sv[c]));
    }
    if (a.output_unsigned) {
        r.lo = 0;
        r.hi = (int64_t(1) << bit_width(out_t)) - 1;
    } else {
        auto [lo, hi] = int_range(out_t);
        r.lo = lo;
        r.hi = hi;
    }
    r.out_bytes = int32_t(dtype_size(out_t));
    return p;
}

// Bounds of CLAMP, src/ops/elementwise.rs:314-343, for integer data.
struct ClampPrep {
    int64_t lo, hi;
};

ClampPrep prepare_clamp_int(const ExecState& st, const Operator& op, const Tensor& input)
{
    const std::string OP = "CLAMP";
    if (op.attr.kind != AttrKind::Clamp)
        throw invalid(OP, "missing attribute");
    if (op.attr.nan_mode == NAN_UNKNOWN)
        throw invalid(OP, "nan_mode must be PROPAGATE or IGNORE");
    const DType t = input.dtype();
    StoragePtr mn, mx;
    try {
        mn = storage_from_raw_bytes(t, op.attr.min_val.data(), op.attr.min_val.size(), 1);
        mx = storage_from_raw_bytes(t, op.attr.max_val.data(), op.attr.max_val.size(), 1);
    } catch (const Error&) {
        throw invalid(OP, "malformed min/max");
    }
    expect_operands(op, OP, 1, 1);
    if (t != DT_INT8 && t != DT_INT16)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported dtype " + dtype_name(t));
    Tensor a, b;
    a.data = mn;
    b.data = mx;
    ClampPrep c{int_values(a)[0], int_values(b)[0]};
    if (c.hi < c.lo)
        throw invalid(OP, "max_val must not be smaller than min_val");
    check_finish(st, OP, op.outputs[0], input.shape, t);
    return c;
}

// A convolution whose int8 RESCALE result feeds a quantised residual, with
// its launch held back (the result is a virtual tensor carrying this): the
// ADD of the residual launches it with the residual in its epilogue when
// conv_i8_residual_ok admits the three RESCALEs; `launch` returns false
// otherwise (nothing launched).
struct ConvResRecipe {
    std::function<bool(void* out, const RescaleDev& ra, const RescaleDev& rb, const RescaleDev& ro, bool cacheable,
                       const int8_t* skip, uint32_t* err, hipStream_t s)>
        launch;
};
constexpr int AUX_CONV_RES = 101;

// The RESCALE (and CLAMP) that follow an int32 producer, prepared for a
// fused epilogue; nullopt when the chain cannot be fused.
struct FusedTail {
    const Operator* rop = nullptr;
    const Operator* cop = nullptr;
    RescalePrep rp;
};

std::optional<FusedTail> plan_tail(const ExecState& st, size_t head, const Shape& shape, DType head_t = DT_INT32)
{
    if (!st.opts.fusion || !st.plan)
        return std::nullopt;
    const int j = st.plan->rescale_after[head];
    if (j < 0)
        return std::nullopt;
    const Operator& rop = st.block->operators[j];
    if (rop.attr.kind != AttrKind::Rescale || rop.inputs.size() != 5 || rop.outputs.size() != 1)
        return std::nullopt;
    TensorPtr ops[4];
    for (int i = 0; i < 4; i++)
        if (!(ops[i] = st.resolve(rop.inputs[1 + i])))
            return std::nullopt;
    Tensor tmp;
    tmp.name = rop.inputs[0];
    tmp.shape = shape;
    tmp.data = std::make_shared<Storage>();
    tmp.data->dtype = head_t;
    tmp.data->count = shape_count(shape);
    FusedTail f;
    f.rop = &rop;
    try {
        f.rp = prepare_rescale(st, rop, tmp, ops[0], ops[1], ops[2], ops[3]);
    } catch (const Error&) {
        return std::nullopt;
    }
    const int k = st.plan->clamp_after[j];
    if (k >= 0) {
        const Operator& cop = st.block->operators[k];
        Tensor rt;
        rt.shape = shape;
        rt.data = std::make_shared<Storage>();
        rt.data->dtype = f.rp.out_t;
        rt.data->count = shape_count(shape);
        try {
            if (!cop.inputs.empty() && cop.inputs[0] == rop.outputs[0]) {
                ClampPrep c = prepare_clamp_int(st, cop, rt);
                f.cop = &cop;
                f.rp.rs.has_clamp = 1;
                f.rp.rs.clamp_lo = c.lo;
                f.rp.rs.clamp_hi = c.hi;
            }
        } catch (const Error&) {
            f.cop = nullptr;
        }
    }
    return f;
}

// Register the outputs of a fused chain: the head's int32 result and (when
// a CLAMP follows) the RESCALE result become virtual tensors recomputed on
// demand; the last output is the one the fused kernel wrote.
void finish_fused(ExecState& st, const std::string& head_out, const Shape& shape, const FusedTail& f,
                  const TensorPtr& final_out, std::function<void(Storage&)> head_fill, DType head_t = DT_INT32)
{
    auto head = virtual_output(head_out, shape, head_t, std::move(head_fill));
    st.set(head);
    if (f.cop) {
        RescalePrep rp = f.rp;
        rp.rs.has_clamp = 0;
        auto src = head;
        const ElemCode he = elem_code(head_t);
        auto mid = virtual_output(f.rop->outputs[0], shape, rp.out_t, [src, rp, he](Storage& out) {
            Stream& s = thread_stream();
            const void* x = src->data->device_in();
            kern::rescale(rp.rs, he, x, out.count, out.device_out(), s.err, s.s);
        });
        st.pending[f.rop->outputs[0]] = mid;
        st.pending[f.cop->outputs[0]] = make_tensor(f.cop->outputs[0], shape, final_out->data);
    } else {
        st.pending[f.rop->outputs[0]] = make_tensor(f.rop->outputs[0], shape, final_out->data);
    }
}

// ---------------------------------------------------------------------------
// CONST, CONST_SHAPE, IDENTITY (src/ops/data_nodes.rs:6-37)
// ---------------------------------------------------------------------------
void eval_const(ExecState& st, const Operator& op)
{
    if (op.outputs.empty())
        throw Error(ERR_GRAPH, "CONST op has no output");
    const std::string& out = op.outputs[0];
    const TensorDef* def = st.find_def(out);
    if (!def)
        throw Error(ERR_TENSOR_NOT_FOUND, out);
    st.set(make_tensor(out, shape_from_ir(def->shape), st.consts->get(*def)));
}

void eval_identity(ExecState& st, const Operator& op)
{
    if (op.inputs.empty())
        throw Error(ERR_GRAPH, "IDENTITY op has no input");
    if (op.outputs.empty())
        throw Error(ERR_GRAPH, "IDENTITY op has no output");
    auto in = st.get(op.inputs[0]);
    st.set(make_tensor(op.outputs[0], in->shape, in->data));
}

// ---------------------------------------------------------------------------
// RESHAPE, TRANSPOSE (src/ops/data_layout.rs:163-177, :246-273)
// ---------------------------------------------------------------------------
void eval_reshape(ExecState& st, const Operator& op)
{
    const std::string OP = "RESHAPE";
    expect_operands(op, OP, 2, 1);
    auto in = st.get(op.inputs[0]);
    auto sh = st.get(op.inputs[1]);
    if (!dtype_is_int(sh->dtype()) && sh->dtype() != DT_SHAPE)
        throw invalid(OP, "operand '" + op.inputs[1] + "' must be a shape, got " + dtype_name(sh->dtype()));
    std::vector<int64_t> ns = int_values(*sh);
    for (int64_t d : ns)
        if (d < 0)
            throw invalid(OP, "shape " + shape_str(ns) + " must be non-negative");
    Shape out(ns.begin(), ns.end());
    if (shape_count(out) != shape_count(in->shape))
        throw Error(ERR_SHAPE_MISMATCH, OP + ": cannot reshape " + shape_str(in->shape) + " to " + shape_str(out));
    check_finish(st, OP, op.outputs[0], out, in->dtype());
    st.set(make_tensor(op.outputs[0], out, in->data));  // same elements, no copy
}

void eval_transpose(ExecState& st, const Operator& op)
{
    const std::string OP = "TRANSPOSE";
    if (op.attr.kind != AttrKind::Transpose)
        throw invalid(OP, "missing attribute");
    expect_operands(op, OP, 1, 1);
    auto in = st.get(op.inputs[0]);
    if (in->shape.empty())
        throw Error(ERR_SHAPE_MISMATCH, OP + ": input must have rank at least 1");
    const size_t rank = in->shape.size();
    const auto& perms = op.attr.perms;
    std::vector<bool> used(rank, false);
    for (int32_t p : perms) {
        if (p < 0 || size_t(p) >= rank || used[p])
            throw invalid(OP, "perms must be a permutation of 0.." + std::to_string(rank));
        used[p] = true;
    }
    if (perms.size() != rank)
        throw invalid(OP, "perms must have " + std::to_string(rank) + " entries");
    Shape out(rank);
    std::vector<int64_t> strides(rank, 1), perm_strides(rank);
    for (int d = int(rank) - 2; d >= 0; d--)
        strides[d] = strides[d + 1] * in->shape[d + 1];
    for (size_t d = 0; d < rank; d++) {
        out[d] = in->shape[perms[d]];
        perm_strides[d] = strides[perms[d]];
    }
    check_finish(st, OP, op.outputs[0], out, in->dtype());
    if (rank > 6)
        throw Error(ERR_SHAPE_MISMATCH, OP + ": rank above 6");
    auto o = new_output(op.outputs[0], out, in->dtype());
    const int64_t n = shape_count(out);
    if (n > 0)
        kern::transpose(in->data->device_in(), o->data->device_out(), int32_t(dtype_size(in->dtype())), int32_t(rank),
                        out.data(), perm_strides.data(), n, st.s());
    st.set(o);
}

// ---------------------------------------------------------------------------
// CONV2D / DEPTHWISE_CONV2D (src/ops/conv.rs:398-524)
// ---------------------------------------------------------------------------
struct ConvGeom {
    int64_t n, ih, iw, ic, oc, m, kh, kw, oh, ow;
    int64_t pt, pl, sy, sx, dy, dx;
    Shape out_shape;
};

int64_t output_extent(const std::string& op, int64_t in, int32_t pb, int32_t pa, int64_t k, int32_t d, int32_t s)
{
    const int64_t full = in - 1 + pb + pa - (k - 1) * d;
    if (full % s != 0)
        throw invalid(op, "parameters must yield exact integer output dimensions");
    const int64_t out = full / s + 1;
    if (out < 1)
        throw invalid(op, "output dimension " + std::to_string(out) + " must be positive");
    return out;
}

void check_conv_attributes(const std::string& op, const OpAttribute& a)
{
    if (a.pad.size() != 4 || a.stride.size() != 2 || a.dilation.size() != 2)
        throw invalid(op, "pad must have 4 elements, stride and dilation 2");
    for (int32_t p : a.pad)
        if (p < 0)
            throw invalid(op, "pad must be non-negative");
    for (int32_t s : a.stride)
        if (s < 1)
            throw invalid(op, "stride must be at least 1");
    for (int32_t d : a.dilation)
        if (d < 1)
            throw invalid(op, "dilation must be at least 1");
}

ConvGeom conv_geometry(const std::string& op, bool depthwise, const Tensor& in, const Tensor& w, const OpAttribute& a)
{
    expect_rank(op, "input", in, 4);
    expect_rank(op, "weight", w, 4);
    check_conv_attributes(op, a);
    ConvGeom g{};
    g.n = in.shape[0];
    g.ih = in.shape[1];
    g.iw = in.shape[2];
    g.ic = in.shape[3];
    if (depthwise) {
        g.kh = w.shape[0];
        g.kw = w.shape[1];
        if (w.shape[2] != g.ic)
            throw Error(ERR_SHAPE_MISMATCH, op + ": weight channels " + std::to_string(w.shape[2]) +
                                                " != input channels " + std::to_string(g.ic));
        g.m = w.shape[3];
        g.oc = g.ic * g.m;
    } else {
        if (w.shape[3] != g.ic)
            throw Error(ERR_SHAPE_MISMATCH, op + ": weight input channels " + std::to_string(w.shape[3]) +
                                                " != input channels " + std::to_string(g.ic));
        g.oc = w.shape[0];
        g.kh = w.shape[1];
        g.kw = w.shape[2];
        g.m = 1;
    }
    g.oh = output_extent(op, g.ih, a.pad[0], a.pad[1], g.kh, a.dilation[0], a.stride[0]);
    g.ow = output_extent(op, g.iw, a.pad[2], a.pad[3], g.kw, a.dilation[1], a.stride[1]);
    g.pt = a.pad[0];
    g.pl = a.pad[2];
    g.sy = a.stride[0];
    g.sx = a.stride[1];
    g.dy = a.dilation[0];
    g.dx = a.dilation[1];
    g.out_shape = {g.n, g.oh, g.ow, g.oc};
    return g;
}

bool conv2d_types(DType i, DType w, DType acc, DType out)
{
    auto fp = [](DType t, std::initializer_list<DType> ok) {
        if (is_fp8(t))
            return true;
        for (DType o : ok)
            if (o == t)
                return true;
        return false;
    };
    if (i == DT_INT8 && (w == DT_INT8 || w == DT_INT4) && acc == DT_INT32 && out == DT_INT32)
        return true;
    if (i == DT_INT16 && w == DT_INT8 && acc == DT_INT48 && out == DT_INT48)
        return true;
    if (acc == DT_FP32 && out == DT_FP32)
        return fp(i, {DT_FP16, DT_BF16, DT_FP32}) && fp(w, {DT_FP16, DT_BF16, DT_FP32});
    if ((acc == DT_FP16 || acc == DT_FP32) && out == DT_FP16)
        return fp(i, {DT_FP16}) && fp(w, {DT_FP16});
    if ((acc == DT_BF16 || acc == DT_FP32) && out == DT_BF16)
        return fp(i, {DT_BF16}) && fp(w, {DT_BF16});
    return false;
}

bool standard_types(DType i, DType w, DType acc, DType out)
{
    if (i == DT_INT8 && (w == DT_INT8 || w == DT_INT4) && acc == DT_INT32 && out == DT_INT32)
        return true;
    if (i == DT_INT16 && w == DT_INT8 && acc == DT_INT48 && out == DT_INT48)
        return true;
    if (i == DT_FP16 && w == DT_FP16 && (acc == DT_FP16 || acc == DT_FP32) && out == DT_FP16)
        return true;
    if (i == DT_BF16 && w == DT_BF16 && acc == DT_FP32 && out == DT_BF16)
        return true;
    if (i == DT_FP32 && w == DT_FP32 && acc == DT_FP32 && out == DT_FP32)
        return true;
    if ((i == DT_FP8E4M3 && w == DT_FP8E4M3) || (i == DT_FP8E5M2 && w == DT_FP8E5M2))
        return (acc == DT_FP16 && out == DT_FP16) || (acc == DT_FP32 && out == DT_FP32);
    return false;
}

AccKind float_acc(DType acc) { return acc == DT_FP16 ? ACC_F16 : (acc == DT_BF16 ? ACC_BF16 : ACC_F32); }

void eval_conv(ExecState& st, const Operator& op, size_t index, bool depthwise)
{
    const std::string OP = depthwise ? "DEPTHWISE_CONV2D" : "CONV2D";
    if (op.attr.kind != (depthwise ? AttrKind::DepthwiseConv2d : AttrKind::Conv2d))
        throw invalid(OP, "missing attribute");
    expect_operands(op, OP, 5, 1);
    auto input = st.get(op.inputs[0]);
    auto weight = st.get(op.inputs[1]);
    auto bias = st.get(op.inputs[2]);
    auto in_zp = single_value(OP, "input_zp", st.get(op.inputs[3]));
    auto w_zp = single_value(OP, "weight_zp", st.get(op.inputs[4]));
    const std::string& out_name = op.outputs[0];

    expect_rank(OP, "bias", *bias, 1);
    ConvGeom g = conv_geometry(OP, depthwise, *input, *weight, op.attr);
    const int64_t bc = bias->shape[0];
    if (bc != g.oc && bc != 1)
        throw Error(ERR_SHAPE_MISMATCH, OP + ": bias channels " + std::to_string(bc) +
                                            " must be 1 or match output channels " + std::to_string(g.oc));
    const DType in_t = input->dtype(), w_t = weight->dtype(), out_t = bias->dtype(), acc_t = op.attr.acc_type;
    auto declared = check_declared_output(st, OP, out_name, g.out_shape);
    if (declared && *declared != out_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": output dtype " + dtype_name(*declared) + " does not match bias dtype " +
                                            dtype_name(out_t));
    if (!(depthwise ? standard_types : conv2d_types)(in_t, w_t, acc_t, out_t))
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported types input=" + dtype_name(in_t) + " weight=" +
                                            dtype_name(w_t) + " acc=" + dtype_name(acc_t) + " output=" +
                                            dtype_name(out_t));
    if (in_zp->dtype() != in_t || w_zp->dtype() != w_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": zero points must match input/weight dtypes");

    const bool is_int = dtype_is_int(acc_t);
    int64_t izp = 0, wzp = 0;
    float fizp = 0.f, fwzp = 0.f;
    if (is_int) {
        izp = int_values(*in_zp)[0];
        wzp = int_values(*w_zp)[0];
        if (izp != 0 && in_t != DT_INT8)
            throw invalid(OP, "input zero point must be zero for non-int8 input");
        if (wzp != 0 && w_t != DT_INT8)
            throw invalid(OP, "weight zero point must be zero for non-int8 weight");
    } else {
        fizp = float(float_values(*in_zp)[0]);
        fwzp = float(float_values(*w_zp)[0]);
        if (fizp != 0.0f || fwzp != 0.0f)
            throw invalid(OP, "zero points must be zero for floating-point operands");
    }

    const int64_t count = shape_count(g.out_shape);
    const int64_t K = g.kh * g.kw * (depthwise ? 1 : g.ic);
    const bool i8 = is_int && acc_t == DT_INT32 && in_t == DT_INT8;
    const bool mfma_int = i8 && !depthwise;
    // int8 depthwise: the MFMA kernel (ic % 16 == 0, <= 12 taps) or the VALU
    // kernel (ic % 4 == 0, small kernels).
    const bool dw_int = i8 && depthwise && g.m == 1 &&
                        (depthwise_i8_supported(int(g.kh), int(g.kw), int(g.ic)) ||
                         (g.ic % 16 == 0 && g.kh * g.kw <= 12));
    const bool mfma_float = !is_int && !depthwise && !st.opts.strict_float && acc_t == DT_FP32 &&
                            ((in_t == DT_BF16 && w_t == DT_BF16) || (in_t == DT_FP16 && w_t == DT_FP16));

    auto sizes_ok = [&]() {
        return g.n * g.ih * g.iw * g.ic < (int64_t(1) << 31) && count < (int64_t(1) << 31) && K < (int64_t(1) << 30);
    };

    if ((mfma_int || dw_int) && sizes_ok()) {
        const void* x = input->data->device_in();
        const void* w = weight->data->device_in();
        // Weight and bias are graph constants: derived data may be cached.
        const bool w_const = st.is_const(op.inputs[1]);
        const bool wb_const = w_const && st.is_const(op.inputs[2]);
        ConvI8Desc fd;
        bool fast = false;
        if (mfma_int || dw_int) {
            fd.x = static_cast<const int8_t*>(x);
            fd.w = static_cast<const int8_t*>(w);
            fd.bias = static_cast<const int32_t*>(bias->data->device_in());
            fd.bias_len = int32_t(bc);
            fd.n = int32_t(g.n);
            fd.ih = int32_t(g.ih);
            fd.iw = int32_t(g.iw);
            fd.ic = int32_t(g.ic);
            fd.oc = int32_t(g.oc);
            fd.kh = int32_t(g.kh);
            fd.kw = int32_t(g.kw);
            fd.oh = int32_t(g.oh);
            fd.ow = int32_t(g.ow);
            fd.pt = int32_t(g.pt);
            fd.pl = int32_t(g.pl);
            fd.sy = int32_t(g.sy);
            fd.sx = int32_t(g.sx);
            fd.dy = int32_t(g.dy);
            fd.dx = int32_t(g.dx);
            fd.zp_x = int32_t(izp);
            fd.zp_w = int32_t(wzp);
            fd.depthwise = depthwise ? 1 : 0;
            fast = conv_i8_fast_supported(fd);
        }
        // Per-channel weight sums for the generic kernel, needed when the
        // input zero point is not 0.
        const int32_t* wsum = nullptr;
        StoragePtr wsum_keep;
        if (izp != 0 && mfma_int) {
            Storage& ws = *weight->data;
            auto make = [&]() {
                auto s = make_device_storage(DT_INT32, g.oc);
                weight_sums_i8(static_cast<const int8_t*>(ws.device_in()), int32_t(g.oc), int32_t(K),
                               static_cast<int32_t*>(s->device_out()), st.s());
                return s;
            };
            wsum_keep = st.is_const(op.inputs[1]) ? cached_aux(ws, AUX_WSUM, make) : make();
            wsum = static_cast<const int32_t*>(wsum_keep->device_in());
        }
        GemmDesc gd;
        DepthwiseDesc dd{};
        if (mfma_int) {
            gd.is_conv = 1;
            gd.elem = ELEM_I8;
            gd.n = int32_t(g.n);
            gd.ih = int32_t(g.ih);
            gd.iw = int32_t(g.iw);
            gd.ic = int32_t(g.ic);
            gd.oc = int32_t(g.oc);
            gd.kh = int32_t(g.kh);
            gd.kw = int32_t(g.kw);
            gd.oh = int32_t(g.oh);
            gd.ow = int32_t(g.ow);
            gd.pt = int32_t(g.pt);
            gd.pl = int32_t(g.pl);
            gd.sy = int32_t(g.sy);
            gd.sx = int32_t(g.sx);
            gd.dy = int32_t(g.dy);
            gd.dx = int32_t(g.dx);
            gd.zp_x = int32_t(izp);
            gd.zp_w = int32_t(wzp);
            gd.wsum = wsum;
            gd.bias = bias->data->device_in();
            gd.bias_len = int32_t(bc);
        } else {
            dd.n = int32_t(g.n);
            dd.ih = int32_t(g.ih);
            dd.iw = int32_t(g.iw);
            dd.c = int32_t(g.ic);
            dd.kh = int32_t(g.kh);
            dd.kw = int32_t(g.kw);
            dd.oh = int32_t(g.oh);
            dd.ow = int32_t(g.ow);
            dd.pt = int32_t(g.pt);
            dd.pl = int32_t(g.pl);
            dd.sy = int32_t(g.sy);
            dd.sx = int32_t(g.sx);
            dd.dy = int32_t(g.dy);
            dd.dx = int32_t(g.dx);
            dd.zp_x = int32_t(izp);
            dd.zp_w = int32_t(wzp);
            dd.bias = static_cast<const int32_t*>(bias->data->device_in());
            dd.bias_len = int32_t(bc);
        }
        // Keep the operands alive for a later recomputation of a fused-away
        // int32 output.
        auto launch = [gd, dd, mfma_int, fast, fd, w_const, wb_const, x, w, input, weight, bias, wsum_keep](
                          void* out, const RescaleDev* rs, bool rs_const, uint32_t* err, hipStream_t s) {
            if (fast && (!rs || conv_i8_fast_epilogue_ok(*rs))) {
                auto tab = conv_i8_table_for(fd, *weight->data, bias->data.get(), rs, wb_const && (!rs || rs_const), s);
                auto wp = conv_i8_wpack_for(fd, *weight->data, w_const, s);
                ConvI8Desc f = fd;
                f.wpack = wp ? static_cast<const int8_t*>(wp->device_in()) : nullptr;
                f.range_safe = tab->scale_range_safe;
                conv_i8_fast(f, tab->device_in(), rs, out, err, s);
                return;
            }
            if (mfma_int && !fast && (!rs || conv_i8_fast_epilogue_ok(*rs)) &&
                int64_t(fd.n) * fd.oh * fd.ow * conv_i8_im2col_kp(fd) < (int64_t(1) << 31)) {
                // Channels or geometry the tiled kernels do not take: a
                // pointwise GEMM over the materialised im2col.
                auto tab = conv_i8_table_for(fd, *weight->data, bias->data.get(), rs, wb_const && (!rs || rs_const), s);
                {
                    // A 1x1 convolution over 8 mod 16 channels: the streaming
                    // pointwise kernel reads the rows as they are.
                    ConvI8Desc sd = fd;
                    sd.range_safe = tab->scale_range_safe;
                    if (conv_i8_pointwise_stream(sd, tab->device_in(), rs, out, err, s))
                        return;
                }
                const int32_t K = fd.kh * fd.kw * fd.ic, kp = conv_i8_im2col_kp(fd);
                auto wp = derived_i8(*weight->data, "conv_i8_rowpad:" + std::to_string(kp), int64_t(fd.oc) * kp,
                                     w_const, s, [&](void* dst) {
                                         conv_i8_rowpad(fd.w, fd.oc, K, kp, static_cast<int8_t*>(dst), s);
                                     });
                if (kp == 32) {
                    // A 3-channel 3x3 stem: the im2col is built in LDS.
                    ConvI8Desc sd = fd;
                    sd.range_safe = tab->scale_range_safe;
                    if (conv_i8_stem(sd, tab->device_in(), static_cast<const int8_t*>(wp->device_in()), rs, out, err, s))
                        return;
                }
                auto xcol = make_device_storage(DT_INT8, int64_t(fd.n) * fd.oh * fd.ow * kp);
                conv_i8_im2col(fd, static_cast<int8_t*>(xcol->device_out()), s);
                ConvI8Desc p = fd;
                p.x = static_cast<const int8_t*>(xcol->device_in());
                p.w = static_cast<const int8_t*>(wp->device_in());
                p.ih = fd.oh;
                p.iw = fd.ow;
                p.ic = kp;
                p.kh = p.kw = 1;
                p.pt = p.pl = 0;
                p.sy = p.sx = p.dy = p.dx = 1;
                p.wpack = nullptr;
                p.range_safe = tab->scale_range_safe;
                conv_i8_fast(p, tab->device_in(), rs, out, err, s);
                return;
            }
            if (fast && !mfma_int && !depthwise_i8_supported(fd.kh, fd.kw, fd.ic)) {
                // A RESCALE the fused epilogue does not take, on a depthwise
                // shape only the MFMA kernel handles: int32 result, then the
                // standalone RESCALE (+CLAMP) kernel.
                auto tab = conv_i8_table_for(fd, *weight->data, bias->data.get(), nullptr, wb_const, s);
                auto tmp = make_device_storage(DT_INT32, int64_t(fd.n) * fd.oh * fd.ow * fd.oc);
                conv_i8_fast(fd, tab->device_in(), nullptr, tmp->device_out(), err, s);
                kern::rescale(*rs, E_I32, tmp->device_in(), tmp->count, out, err, s);
                return;
            }
            if (mfma_int) {
                GemmDesc d = gd;
                if (rs) {
                    d.epi = EPI_RESCALE;
                    d.rs = *rs;
                }
                kern::gemm(d, x, w, out, err, s);
            } else {
                DepthwiseDesc d = dd;
                if (rs) {
                    d.epi = EPI_RESCALE;
                    d.rs = *rs;
                }
                kern::depthwise_i8(d, static_cast<const int8_t*>(x), static_cast<const int8_t*>(w), out, err, s);
            }
        };
        if (auto tail = plan_tail(st, index, g.out_shape)) {
            if (fast && count > 0 && !tail->cop && st.plan->residual_head[index] && tail->rp.out_t == DT_INT8) {
                // The result y only feeds a residual: hold the launch back
                // for the ADD, which may fold the residual into it.
                const bool rs_const = st.is_const(tail->rop->inputs[1]) && st.is_const(tail->rop->inputs[2]);
                const RescaleDev rsj = tail->rp.rs;
                auto keep = tail->rp.params;
                auto head = virtual_output(out_name, g.out_shape, DT_INT32, [launch, keep](Storage& o) {
                    Stream& s = thread_stream();
                    launch(o.device_out(), nullptr, false, s.err, s.s);
                });
                st.set(head);
                auto y = virtual_output(tail->rop->outputs[0], g.out_shape, DT_INT8,
                                        [launch, keep, rsj, rs_const](Storage& o) {
                                            Stream& s = thread_stream();
                                            launch(o.device_out(), &rsj, rs_const, s.err, s.s);
                                        });
                auto recipe = std::make_shared<ConvResRecipe>();
                recipe->launch = [fd, weight, bias, w_const, wb_const, rsj, rs_const, keep, x](
                                     void* out, const RescaleDev& ra, const RescaleDev& rb, const RescaleDev& ro,
                                     bool cacheable, const int8_t* skip, uint32_t* err, hipStream_t s) {
                    if (!conv_i8_residual_ok(fd, rsj, ra, rb, ro, skip))
                        return false;
                    (void)x;
                    auto tab = conv_i8_table_for(fd, *weight->data, bias->data.get(), &rsj, wb_const && rs_const, s);
                    char key[192];
                    std::snprintf(key, sizeof key, "conv_i8_res:%p:%p:%p:%p:%p:%p:%d:%d:%d:%d:%d:%d:%lld",
                                  static_cast<const void*>(ra.mult), static_cast<const void*>(ra.shift),
                                  static_cast<const void*>(rb.mult), static_cast<const void*>(rb.shift),
                                  static_cast<const void*>(ro.mult), static_cast<const void*>(ro.shift),
                                  ra.per_channel, rb.per_channel, ro.per_channel, ra.rounding, rb.rounding,
                                  ro.rounding, static_cast<long long>(ro.out_zp));
                    auto rtab = derived_i8(*weight->data, key, int64_t(fd.oc) * CONV_I8_RES_WORDS * 4,
                                           w_const && cacheable, s, [&](void* dst) {
                                               conv_i8_residual_table(ra, rb, ro, fd.oc, dst, s);
                                           });
                    ConvI8Desc f = fd;
                    f.range_safe = tab->scale_range_safe;
                    f.res_skip = skip;
                    f.res_tab = rtab->device_in();
                    f.res_za = int32_t(ra.in_zp);
                    f.res_zb = int32_t(rb.in_zp);
                    f.res_clo = int32_t(ro.has_clamp ? std::max<int64_t>(ro.clamp_lo, ro.lo) : ro.lo);
                    f.res_chi = int32_t(ro.has_clamp ? std::min<int64_t>(ro.clamp_hi, ro.hi) : ro.hi);
                    conv_i8_fast(f, tab->device_in(), &rsj, out, err, s);
                    return true;
                };
                y->data->aux = std::shared_ptr<Storage>(recipe, reinterpret_cast<Storage*>(recipe.get()));
                y->data->aux_kind = AUX_CONV_RES;
                st.pending[tail->rop->outputs[0]] = y;
                return;
            }
            const DType final_t = tail->rp.out_t;
            auto fin = new_output(tail->cop ? tail->cop->outputs[0] : tail->rop->outputs[0], g.out_shape, final_t);
            const bool rs_const =
                st.is_const(tail->rop->inputs[1]) && st.is_const(tail->rop->inputs[2]);
            if (count > 0)
                launch(fin->data->device_out(), &tail->rp.rs, rs_const, st.err(), st.s());
            auto keep = tail->rp.params;
            finish_fused(st, out_name, g.out_shape, *tail, fin, [launch, keep](Storage& o) {
                Stream& s = thread_stream();
                if (o.count > 0)
                    launch(o.device_out(), nullptr, false, s.err, s.s);
                else
                    o.device_out();
            });
            return;
        }
        auto out = new_output(out_name, g.out_shape, DT_INT32);
        void* od = out->data->device_out();
        if (count > 0)
            launch(od, nullptr, false, st.err(), st.s());
        st.set(out);
        return;
    }

    if (mfma_float && sizes_ok()) {
        // Bias as f32 values, kept with a constant bias tensor (rebuilt per
        // run otherwise: the caller may rewrite a wrapped buffer).
        Storage& bs = *bias->data;
        auto make_bf = [&]() {
            std::vector<double> v = float_values(*bias);
            std::vector<float> f(v.begin(), v.end());
            auto h = make_host_storage(DT_FP32, int64_t(f.size()), f.data());
            h->shared_const = st.is_const(op.inputs[2]);
            return h;
        };
        auto bf = st.is_const(op.inputs[2]) ? cached_aux(bs, AUX_F32, make_bf) : make_bf();
        GemmDesc gd;
        gd.is_conv = 1;
        gd.elem = in_t == DT_BF16 ? ELEM_BF16 : ELEM_F16;
        gd.n = int32_t(g.n);
        gd.ih = int32_t(g.ih);
        gd.iw = int32_t(g.iw);
        gd.ic = int32_t(g.ic);
        gd.oc = int32_t(g.oc);
        gd.kh = int32_t(g.kh);
        gd.kw = int32_t(g.kw);
        gd.oh = int32_t(g.oh);
        gd.ow = int32_t(g.ow);
        gd.pt = int32_t(g.pt);
        gd.pl = int32_t(g.pl);
        gd.sy = int32_t(g.sy);
        gd.sx = int32_t(g.sx);
        gd.dy = int32_t(g.dy);
        gd.dx = int32_t(g.dx);
        gd.bias = bf->device_in();
        gd.bias_len = int32_t(bc);
        gd.epi = EPI_FLOAT;
        gd.out_fmt = FloatFmt(fmt_code(out_t));
        auto out = new_output(out_name, g.out_shape, out_t);
        void* od = out->data->device_out();
        const void* xd = input->data->device_in();
        const void* wd = weight->data->device_in();
        const bool pw = g.kh == 1 && g.kw == 1 && g.sy == 1 && g.sx == 1 && g.pt == 0 && g.pl == 0 && g.ih == g.oh &&
                        g.iw == g.ow;
        if (count > 0 && pw && kern::gemm_f16_supported(1, g.n * g.oh * g.ow, g.oc, g.ic, false, xd, wd)) {
            // 1x1 convolution: NHWC rows x OHWI rows on the dedicated GEMM.
            GemmF16Desc fd;
            fd.m = int32_t(g.n * g.oh * g.ow);
            fd.n = int32_t(g.oc);
            fd.k = int32_t(g.ic);
            fd.elem = gd.elem;
            fd.b_kn = false;
            fd.bias = gd.bias;
            fd.bias_len = gd.bias_len;
            fd.out_fmt = gd.out_fmt;
            kern::gemm_f16(fd, xd, wd, od, st.s());
        } else if (count > 0) {
            kern::ConvF16Desc hd;
            hd.x = xd;
            hd.w = wd;
            hd.elem = gd.elem;
            hd.n = gd.n;
            hd.ih = gd.ih;
            hd.iw = gd.iw;
            hd.ic = gd.ic;
            hd.oc = gd.oc;
            hd.kh = gd.kh;
            hd.kw = gd.kw;
            hd.oh = gd.oh;
            hd.ow = gd.ow;
            hd.pt = gd.pt;
            hd.pl = gd.pl;
            hd.sy = gd.sy;
            hd.sx = gd.sx;
            hd.dy = gd.dy;
            hd.dx = gd.dx;
            hd.bias = static_cast<const float*>(gd.bias);
            hd.bias_len = gd.bias_len;
            hd.out_fmt = gd.out_fmt;
            const int64_t wpb = kern::conv_f16_halo_wpack_bytes(hd);
            if (wpb > 0) {
                // Stride-1 convolution on the halo kernel, with its packed
                // weights cached on a constant weight.
                const bool w_const = st.is_const(op.inputs[1]);
                const std::string key =
                    "conv_f16_wpack:" + std::to_string(wpb) + ":" + std::to_string(kern::conv_f16_halo_block(hd));
                auto wp = derived_i8(*weight->data, key, wpb, w_const, st.s(),
                                     [&](void* dst) { kern::conv_f16_halo_wpack(hd, dst, st.s()); });
                hd.wpack = wp->device_in();
                kern::conv_f16_halo(hd, od, st.s());
            } else {
                kern::gemm(gd, xd, wd, od, st.err(), st.s());
            }
        }
        st.set(out);
        return;
    }

    // int16 x int8 -> INT48 (src/ops/conv.rs:457-473, AccI64) on the int8
    // MFMA kernels. The input as int8 halves, x = 256 hi + lo with lo held as
    // lo - 128: the sum of x (w - zw) is 256 times that of hi plus that of
    // (lo - 128) - (-128), i.e. a second convolution with input zero point
    // -128 (which padding taps also take, so they still add nothing). Each
    // half accumulates in int32 without wrapping while K 255 255 < 2^31; the
    // two combine with the bias in int64, clamped to 48 bits.
    if (is_int && in_t == DT_INT16 && w_t == DT_INT8 && acc_t == DT_INT48 && !depthwise && izp == 0 &&
        K * 65025 < (int64_t(1) << 31) && sizes_ok() && count > 0) {
        const int64_t xcount = g.n * g.ih * g.iw * g.ic;
        auto hi = make_device_storage(DT_INT8, xcount);
        auto lo = make_device_storage(DT_INT8, xcount);
        ConvI8Desc fd;
        fd.x = static_cast<const int8_t*>(hi->device_out());
        fd.w = static_cast<const int8_t*>(weight->data->device_in());
        fd.bias = nullptr;
        fd.bias_len = 1;
        fd.n = int32_t(g.n);
        fd.ih = int32_t(g.ih);
        fd.iw = int32_t(g.iw);
        fd.ic = int32_t(g.ic);
        fd.oc = int32_t(g.oc);
        fd.kh = int32_t(g.kh);
        fd.kw = int32_t(g.kw);
        fd.oh = int32_t(g.oh);
        fd.ow = int32_t(g.ow);
        fd.pt = int32_t(g.pt);
        fd.pl = int32_t(g.pl);
        fd.sy = int32_t(g.sy);
        fd.sx = int32_t(g.sx);
        fd.dy = int32_t(g.dy);
        fd.dx = int32_t(g.dx);
        fd.zp_w = int32_t(wzp);
        if (conv_i8_fast_supported(fd)) {
            hipStream_t s = st.s();
            const bool w_const = st.is_const(op.inputs[1]);
            kern::split_i16(static_cast<const int16_t*>(input->data->device_in()), xcount,
                            static_cast<int8_t*>(hi->device_out()), static_cast<int8_t*>(lo->device_out()), s);
            auto wp = conv_i8_wpack_for(fd, *weight->data, w_const, s);
            fd.wpack = wp ? static_cast<const int8_t*>(wp->device_in()) : nullptr;
            ConvI8Desc dl = fd;
            dl.x = static_cast<const int8_t*>(lo->device_in());
            dl.zp_x = -128;
            auto th = conv_i8_table_for(fd, *weight->data, nullptr, nullptr, w_const, s);
            auto tl = conv_i8_table_for(dl, *weight->data, nullptr, nullptr, w_const, s);
            auto ph = make_device_storage(DT_INT32, count);
            auto pl = make_device_storage(DT_INT32, count);
            conv_i8_fast(fd, th->device_in(), nullptr, ph->device_out(), st.err(), s);
            conv_i8_fast(dl, tl->device_in(), nullptr, pl->device_out(), st.err(), s);
            const int32_t* parts[2] = {static_cast<const int32_t*>(ph->device_in()),
                                       static_cast<const int32_t*>(pl->device_in())};
            const int64_t coef[2] = {256, 1};
            const int64_t* bdev = static_cast<const int64_t*>(bias->data->device_in());
            const int32_t oc = int32_t(g.oc);
            if (auto tail = plan_tail(st, index, g.out_shape, DT_INT48)) {
                // The RESCALE (and CLAMP) after the convolution read the
                // combined values directly; the INT48 tensor is made only if
                // something asks for it.
                auto fin = new_output(tail->cop ? tail->cop->outputs[0] : tail->rop->outputs[0], g.out_shape,
                                      tail->rp.out_t);
                kern::combine_i48_rescale(parts, coef, 2, bdev, int32_t(bc), oc, count, tail->rp.rs,
                                          fin->data->device_out(), st.err(), s);
                auto keep = tail->rp.params;
                finish_fused(
                    st, out_name, g.out_shape, *tail, fin,
                    [ph, pl, bias, bc, oc, count, keep](Storage& o) {
                        Stream& ts = thread_stream();
                        const int32_t* p2[2] = {static_cast<const int32_t*>(ph->device_in()),
                                                static_cast<const int32_t*>(pl->device_in())};
                        const int64_t c2[2] = {256, 1};
                        kern::combine_i48(p2, c2, 2, static_cast<const int64_t*>(bias->data->device_in()),
                                          int32_t(bc), oc, count, static_cast<int64_t*>(o.device_out()), ts.s);
                    },
                    DT_INT48);
                return;
            }
            auto out = new_output(out_name, g.out_shape, DT_INT48);
            kern::combine_i48(parts, coef, 2, bdev, int32_t(bc), oc, count,
                              static_cast<int64_t*>(out->data->device_out()), s);
            st.set(out);
            return;
        }
    }

    // Reference-order kernel for every other combination.
    DirectConvDesc d{};
    d.depthwise = depthwise;
    d.n = int32_t(g.n);
    d.ih = int32_t(g.ih);
    d.iw = int32_t(g.iw);
    d.c = int32_t(g.ic);
    d.m = int32_t(g.m);
    d.oc = int32_t(g.oc);
    d.kh = int32_t(g.kh);
    d.kw = int32_t(g.kw);
    d.oh = int32_t(g.oh);
    d.ow = int32_t(g.ow);
    d.pt = int32_t(g.pt);
    d.pl = int32_t(g.pl);
    d.sy = int32_t(g.sy);
    d.sx = int32_t(g.sx);
    d.dy = int32_t(g.dy);
    d.dx = int32_t(g.dx);
    d.xe = elem_code(in_t);
    d.we = elem_code(w_t);
    d.be = elem_code(out_t);
    d.oe = elem_code(out_t);
    d.acc = is_int ? (acc_t == DT_INT32 ? ACC_I32 : ACC_I64) : float_acc(acc_t);
    d.zp_x = izp;
    d.zp_w = wzp;
    d.fzp_x = fizp;
    d.fzp_w = fwzp;
    d.bias_len = int32_t(bc);
    d.out_fmt = fmt_code(out_t);
    auto out = new_output(out_name, g.out_shape, out_t);
    void* od = out->data->device_out();
    if (count > 0)
        kern::direct_conv(d, input->data->device_in(), weight->data->device_in(), bias->data->device_in(), od, st.s());
    st.set(out);
}

// ---------------------------------------------------------------------------
// MATMUL (src/ops/matmul.rs:98-178)
// ---------------------------------------------------------------------------
bool matmul_types(DType a, DType b, DType out)
{
    if (a == DT_INT8 && b == DT_INT8 && out == DT_INT32)
        return true;
    if (a == DT_INT16 && b == DT_INT16 && out == DT_INT48)
        return true;
    if (a == DT_FP16 && b == DT_FP16 && (out == DT_FP16 || out == DT_FP32))
        return true;
    if (a == DT_BF16 && b == DT_BF16 && out == DT_FP32)
        return true;
    if (a == DT_FP32 && b == DT_FP32 && out == DT_FP32)
        return true;
    if (out == DT_FP16 || out == DT_FP32)
        return is_fp8(a) && is_fp8(b);
    return false;
}

// MATMUL_T's (a, b, output) combinations (src/ops/matmul.rs:40-51): any mix
// of FP8/FP16/BF16/FP32 operands into BF16 or FP32 (FP32 operands need an
// FP32 output), plus the integer pairs and FP16 x FP16 -> FP16.
bool matmul_t_types(DType a, DType b, DType out)
{
    auto fl = [](DType t) { return is_fp8(t) || t == DT_FP16 || t == DT_BF16 || t == DT_FP32; };
    if ((a == DT_INT8 && b == DT_INT8 && out == DT_INT32) || (a == DT_INT16 && b == DT_INT16 && out == DT_INT48) ||
        (a == DT_FP16 && b == DT_FP16 && out == DT_FP16))
        return true;
    if (out == DT_FP32)
        return fl(a) && fl(b);
    if (out == DT_BF16)
        return fl(a) && fl(b) && a != DT_FP32 && b != DT_FP32 && !(a == DT_FP16 && b == DT_FP16);
    return false;
}

DType matmul_default_output(DType a)
{
    switch (a) {
    case DT_INT8: return DT_INT32;
    case DT_INT16: return DT_INT48;
    case DT_FP16:
    case DT_FP8E4M3:
    case DT_FP8E5M2: return DT_FP16;
    default: return DT_FP32;
    }
}

// MATMUL (transposed false) and MATMUL_T (true): b [N,C,W], or b [D,W,C]
// with D = N or 1 (broadcast). src/ops/matmul.rs:98-182.
void eval_matmul(ExecState& st, const Operator& op, size_t index, bool transposed)
{
    const std::string OP = transposed ? "MATMUL_T" : "MATMUL";
    expect_operands(op, OP, 4, 1);
    auto a = st.get(op.inputs[0]);
    auto b = st.get(op.inputs[1]);
    auto a_zp = single_value(OP, "a_zp", st.get(op.inputs[2]));
    auto b_zp = single_value(OP, "b_zp", st.get(op.inputs[3]));
    const std::string& out_name = op.outputs[0];
    expect_rank(OP, "a", *a, 3);
    expect_rank(OP, "b", *b, 3);
    const int64_t n = a->shape[0], h = a->shape[1], c = a->shape[2];
    const int64_t bn = b->shape[0], bc = transposed ? b->shape[2] : b->shape[1];
    const int64_t w = transposed ? b->shape[1] : b->shape[2];
    if (bc != c || (bn != n && !(transposed && bn == 1)))
        throw Error(ERR_SHAPE_MISMATCH, OP + ": b shape " + shape_str(b->shape) + " incompatible with a shape " +
                                            shape_str(a->shape));
    const bool broadcast = bn != n;
    const Shape out_shape = {n, h, w};
    const DType a_t = a->dtype(), b_t = b->dtype();
    const DType out_t = check_declared_output(st, OP, out_name, out_shape).value_or(matmul_default_output(a_t));
    if (!(transposed ? matmul_t_types : matmul_types)(a_t, b_t, out_t))
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported types a=" + dtype_name(a_t) + " b=" + dtype_name(b_t) +
                                            " output=" + dtype_name(out_t));
    if (a_zp->dtype() != a_t || b_zp->dtype() != b_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": zero points must match input dtypes");
    const int64_t count = shape_count(out_shape);
    const bool is_int = dtype_is_int(out_t);
    int64_t azp = 0, bzp = 0;
    if (is_int) {
        azp = int_values(*a_zp)[0];
        bzp = int_values(*b_zp)[0];
        if ((azp != 0 && a_t != DT_INT8) || (bzp != 0 && b_t != DT_INT8))
            throw invalid(OP, "zero points must be zero for non-int8 inputs");
    } else {
        if (float_values(*a_zp)[0] != 0.0 || float_values(*b_zp)[0] != 0.0)
            throw invalid(OP, "zero points must be zero for floating-point inputs");
    }
    const bool small = n * h * c < (int64_t(1) << 31) && n * c * w < (int64_t(1) << 31) && count < (int64_t(1) << 31);
    const bool mfma_int = out_t == DT_INT32 && small;
    const bool mfma_float = !is_int && out_t == DT_FP32 && !st.opts.strict_float && small &&
                            ((a_t == DT_BF16 && b_t == DT_BF16) || (a_t == DT_FP16 && b_t == DT_FP16));
    const void* a_dev = (mfma_int && c % 16 == 0) ? a->data->device_in() : nullptr;
    const void* b_dev = transposed && a_dev ? b->data->device_in() : nullptr;
    if (a_dev && reinterpret_cast<uintptr_t>(a_dev) % 16 == 0 &&
        (!transposed || reinterpret_cast<uintptr_t>(b_dev) % 16 == 0)) {
        // int8: the pointwise tiled kernel, one batch per grid slice, over B
        // as rows of c bytes: MATMUL_T's own layout, or MATMUL's B transposed
        // (cached when B is a graph constant); zero points folded into the
        // accumulator like CONV2D's. A MATMUL_T B shared by every batch
        // makes the batches one problem of n h rows.
        const bool b_const = st.is_const(op.inputs[1]);
        ConvI8Desc fd;
        fd.x = static_cast<const int8_t*>(a_dev);
        fd.bias = nullptr;
        fd.bias_len = 1;
        fd.n = 1;
        fd.ih = fd.oh = int32_t(broadcast ? n * h : h);
        fd.iw = fd.ow = 1;
        fd.ic = int32_t(c);
        fd.oc = int32_t(w);
        fd.zp_x = int32_t(azp);
        fd.zp_w = int32_t(bzp);
        fd.batch = int32_t(broadcast ? 1 : n);
        auto launch = [fd, a, b, b_const, transposed](void* out, const RescaleDev* rs, bool rs_const, uint32_t* err,
                                                      hipStream_t s) {
            ConvI8Desc d = fd;
            if (!transposed && kern::matmul_i8_direct_applies(d.ic, d.oc, d.x, b->data->device_in())) {
                // One kernel, B read in its own layout; the table (no weight
                // sums: the kernel adds the a-zero-point term itself) does not
                // depend on B's values.
                ConvI8Desc td = d;
                td.w = nullptr;
                td.batch = 1;
                auto tab = conv_i8_table_for(td, *b->data, nullptr, rs, !rs || rs_const, s);
                if (kern::matmul_i8_direct(d.x, static_cast<const int8_t*>(b->data->device_in()), d.batch, d.ih,
                                           d.ic, d.oc, d.zp_x, d.zp_w, tab->device_in(), rs, tab->scale_range_safe,
                                           out, err, s))
                    return;
            }
            StoragePtr bt;
            if (transposed) {
                d.w = static_cast<const int8_t*>(b->data->device_in());
            } else {
                bt = derived_i8(*b->data, "matmul_bt", int64_t(d.batch) * d.ic * d.oc, b_const, s, [&](void* dst) {
                    transpose_b_i8(static_cast<const int8_t*>(b->data->device_in()), d.batch, d.ic, d.oc,
                                   static_cast<int8_t*>(dst), s);
                });
                d.w = static_cast<const int8_t*>(bt->device_in());
            }
            auto tab = conv_i8_table_for(d, *b->data, nullptr, rs, b_const && (!rs || rs_const), s);
            d.range_safe = tab->scale_range_safe;
            conv_i8_fast(d, tab->device_in(), rs, out, err, s);
        };
        if (auto tail = plan_tail(st, index, out_shape)) {
            if (conv_i8_fast_epilogue_ok(tail->rp.rs)) {
                auto fin =
                    new_output(tail->cop ? tail->cop->outputs[0] : tail->rop->outputs[0], out_shape, tail->rp.out_t);
                const bool rs_const =
                    st.is_const(tail->rop->inputs[1]) && st.is_const(tail->rop->inputs[2]);
                if (count > 0)
                    launch(fin->data->device_out(), &tail->rp.rs, rs_const, st.err(), st.s());
                auto keep = tail->rp.params;
                finish_fused(st, out_name, out_shape, *tail, fin, [launch, keep](Storage& o) {
                    Stream& s = thread_stream();
                    if (o.count > 0)
                        launch(o.device_out(), nullptr, false, s.err, s.s);
                    else
                        o.device_out();
                });
                return;
            }
        }
        auto out = new_output(out_name, out_shape, DT_INT32);
        if (count > 0)
            launch(out->data->device_out(), nullptr, false, st.err(), st.s());
        st.set(out);
        return;
    }
    const int64_t fbatch = broadcast ? 1 : n, fm = broadcast ? n * h : h;
    if (mfma_float && count > 0 &&
        kern::gemm_f16_supported(fbatch, fm, w, c, !transposed, a->data->device_in(), b->data->device_in())) {
        GemmF16Desc fd;
        fd.batch = int32_t(fbatch);
        fd.m = int32_t(fm);
        fd.n = int32_t(w);
        fd.k = int32_t(c);
        fd.elem = a_t == DT_BF16 ? ELEM_BF16 : ELEM_F16;
        fd.b_kn = !transposed;
        fd.out_fmt = FMT_F32;
        auto out = new_output(out_name, out_shape, out_t);
        kern::gemm_f16(fd, a->data->device_in(), b->data->device_in(), out->data->device_out(), st.s());
        st.set(out);
        return;
    }
    if ((mfma_int || mfma_float) && !transposed) {
        GemmDesc gd;
        gd.is_conv = 0;
        gd.elem = mfma_int ? ELEM_I8 : (a_t == DT_BF16 ? ELEM_BF16 : ELEM_F16);
        gd.batch = int32_t(n);
        gd.h = int32_t(h);
        gd.c = int32_t(c);
        gd.w = int32_t(w);
        gd.zp_x = int32_t(azp);
        gd.zp_w = int32_t(bzp);
        gd.epi = mfma_int ? EPI_I32 : EPI_FLOAT;
        gd.out_fmt = FMT_F32;
        const void* ad = a->data->device_in();
        const void* bd = b->data->device_in();
        if (mfma_int) {
            if (auto tail = plan_tail(st, index, out_shape)) {
                auto fin =
                    new_output(tail->cop ? tail->cop->outputs[0] : tail->rop->outputs[0], out_shape, tail->rp.out_t);
                GemmDesc fd = gd;
                fd.epi = EPI_RESCALE;
                fd.rs = tail->rp.rs;
                void* fo = fin->data->device_out();
                if (count > 0)
                    kern::gemm(fd, ad, bd, fo, st.err(), st.s());
                auto keep = tail->rp.params;
                finish_fused(st, out_name, out_shape, *tail, fin, [gd, ad, bd, a, b, keep](Storage& o) {
                    Stream& s = thread_stream();
                    void* od = o.device_out();
                    if (o.count > 0)
                        kern::gemm(gd, ad, bd, od, s.err, s.s);
                });
                return;
            }
        }
        auto out = new_output(out_name, out_shape, out_t);
        void* od = out->data->device_out();
        if (count > 0)
            kern::gemm(gd, ad, bd, od, st.err(), st.s());
        st.set(out);
        return;
    }
    // int16 x int16 -> INT48 (src/ops/matmul.rs:147-153) on the int8 MFMA
    // kernel: both operands as int8 halves (a = 256 ah + al, b = 256 bh + bl,
    // the lows held minus 128): four int8 products, a low half entering with
    // zero point -128, combined in int64 as 65536 P(hh) + 256 (P(hl) + P(lh))
    // + P(ll) and clamped to 48 bits. Exact while C 255 255 < 2^31.
    if (is_int && a_t == DT_INT16 && out_t == DT_INT48 && small && count > 0 && c % 16 == 0 &&
        c * 65025 < (int64_t(1) << 31)) {
        hipStream_t s = st.s();
        const int64_t acount = n * h * c, bcount = shape_count(b->shape);
        auto ah = make_device_storage(DT_INT8, acount), al = make_device_storage(DT_INT8, acount);
        auto bh = make_device_storage(DT_INT8, bcount), bl = make_device_storage(DT_INT8, bcount);
        kern::split_i16(static_cast<const int16_t*>(a->data->device_in()), acount,
                        static_cast<int8_t*>(ah->device_out()), static_cast<int8_t*>(al->device_out()), s);
        kern::split_i16(static_cast<const int16_t*>(b->data->device_in()), bcount,
                        static_cast<int8_t*>(bh->device_out()), static_cast<int8_t*>(bl->device_out()), s);
        // B halves as rows of c bytes: MATMUL_T's own layout, MATMUL's transposed.
        auto rows = [&](const StoragePtr& half) {
            if (transposed)
                return half;
            auto t = make_device_storage(DT_INT8, bcount);
            transpose_b_i8(static_cast<const int8_t*>(half->device_in()), int32_t(n), int32_t(c), int32_t(w),
                           static_cast<int8_t*>(t->device_out()), s);
            return t;
        };
        const StoragePtr bhr = rows(bh), blr = rows(bl);
        ConvI8Desc fd;
        fd.bias = nullptr;
        fd.bias_len = 1;
        fd.n = 1;
        fd.ih = fd.oh = int32_t(broadcast ? n * h : h);
        fd.iw = fd.ow = 1;
        fd.ic = int32_t(c);
        fd.oc = int32_t(w);
        fd.batch = int32_t(broadcast ? 1 : n);
        auto part = [&](const StoragePtr& x8, const StoragePtr& w8, int32_t zx, int32_t zw) {
            ConvI8Desc d = fd;
            d.x = static_cast<const int8_t*>(x8->device_in());
            d.w = static_cast<const int8_t*>(w8->device_in());
            d.zp_x = zx;
            d.zp_w = zw;
            auto tab = conv_i8_table_for(d, *w8, nullptr, nullptr, false, s);
            auto out = make_device_storage(DT_INT32, count);
            conv_i8_fast(d, tab->device_in(), nullptr, out->device_out(), st.err(), s);
            return out;
        };
        const StoragePtr p[4] = {part(ah, bhr, 0, 0), part(ah, blr, 0, -128), part(al, bhr, -128, 0),
                                 part(al, blr, -128, -128)};
        const int32_t* parts[4];
        for (int k = 0; k < 4; k++)
            parts[k] = static_cast<const int32_t*>(p[k]->device_in());
        const int64_t coef[4] = {65536, 256, 256, 1};
        if (auto tail = plan_tail(st, index, out_shape, DT_INT48)) {
            // The RESCALE (and CLAMP) after the MATMUL read the combined
            // values directly (channels: the columns w).
            auto fin = new_output(tail->cop ? tail->cop->outputs[0] : tail->rop->outputs[0], out_shape,
                                  tail->rp.out_t);
            kern::combine_i48_rescale(parts, coef, 4, nullptr, 1, int32_t(w), count, tail->rp.rs,
                                      fin->data->device_out(), st.err(), s);
            auto keep = tail->rp.params;
            const StoragePtr q0 = p[0], q1 = p[1], q2 = p[2], q3 = p[3];
            finish_fused(
                st, out_name, out_shape, *tail, fin,
                [q0, q1, q2, q3, count, keep](Storage& o) {
                    Stream& ts = thread_stream();
                    const int32_t* p4[4] = {static_cast<const int32_t*>(q0->device_in()),
                                            static_cast<const int32_t*>(q1->device_in()),
                                            static_cast<const int32_t*>(q2->device_in()),
                                            static_cast<const int32_t*>(q3->device_in())};
                    const int64_t c4[4] = {65536, 256, 256, 1};
                    kern::combine_i48(p4, c4, 4, nullptr, 1, 1, count, static_cast<int64_t*>(o.device_out()), ts.s);
                },
                DT_INT48);
            return;
        }
        auto out = new_output(out_name, out_shape, DT_INT48);
        kern::combine_i48(parts, coef, 4, nullptr, 1, 1, count, static_cast<int64_t*>(out->data->device_out()), s);
        st.set(out);
        return;
    }
    DirectMatmulDesc d{};
    d.batch = int32_t(n);
    d.h = int32_t(h);
    d.c = int32_t(c);
    d.w = int32_t(w);
    d.b_transposed = transposed ? 1 : 0;
    d.b_broadcast = broadcast ? 1 : 0;
    d.ae = elem_code(a_t);
    d.be = elem_code(b_t);
    d.oe = elem_code(out_t);
    d.zp_a = azp;
    d.zp_b = bzp;
    if (is_int)
        d.acc = out_t == DT_INT32 ? ACC_I32 : ACC_I64;
    else
        d.acc = out_t == DT_FP16 ? ACC_F16U : (out_t == DT_BF16 ? ACC_BF16U : ACC_F32);
    d.out_fmt = fmt_code(out_t);
    auto out = new_output(out_name, out_shape, out_t);
    void* od = out->data->device_out();
    if (count > 0)
        kern::direct_matmul(d, a->data->device_in(), b->data->device_in(), od, st.s());
    st.set(out);
}

// ---------------------------------------------------------------------------
// AVG_POOL2D (src/ops/pool.rs:17-105, :146-231)
// ---------------------------------------------------------------------------
// PoolGeometry::new (src/ops/pool.rs:30-70): shared by AVG_POOL2D and
// MAX_POOL2D. Fills the geometry fields of a PoolDesc.
PoolDesc pool_geometry(const std::string& OP, const Tensor& input, const std::vector<int32_t>& kernel,
                       const std::vector<int32_t>& stride, const std::vector<int32_t>& pad)
{
    expect_rank(OP, "input", input, 4);
    if (pad.size() != 4 || kernel.size() != 2 || stride.size() != 2)
        throw invalid(OP, "pad must have 4 elements, kernel and stride 2");
    for (int32_t p : pad)
        if (p < 0)
            throw invalid(OP, "pad must be non-negative");
    for (int32_t k : kernel)
        if (k < 1)
            throw invalid(OP, "kernel and stride must be at least 1");
    for (int32_t s : stride)
        if (s < 1)
            throw invalid(OP, "kernel and stride must be at least 1");
    if (pad[0] >= kernel[0] || pad[1] >= kernel[0] || pad[2] >= kernel[1] || pad[3] >= kernel[1])
        throw invalid(OP, "pad must be smaller than kernel");
    const int64_t n = input.shape[0], ih = input.shape[1], iw = input.shape[2], c = input.shape[3];
    if (ih == 0 || iw == 0)
        throw invalid(OP, "input height and width must be positive");
    auto extent = [&](int64_t size, int32_t a, int32_t b, int32_t k, int32_t s) {
        const int64_t full = size + a + b - k;
        if (full < 0 || full % s != 0)
            throw invalid(OP, "parameters must yield exact integer output dimensions");
        return full / s + 1;
    };
    const int64_t oh = extent(ih, pad[0], pad[1], kernel[0], stride[0]);
    const int64_t ow = extent(iw, pad[2], pad[3], kernel[1], stride[1]);
    if (n * ih * iw * c >= (int64_t(1) << 31) || n * oh * ow * c >= (int64_t(1) << 31))
        throw Error(ERR_SHAPE_MISMATCH, OP + ": tensors of 2^31 elements or more are not supported");
    PoolDesc d{};
    d.n = int32_t(n);
    d.ih = int32_t(ih);
    d.iw = int32_t(iw);
    d.c = int32_t(c);
    d.kh = kernel[0];
    d.kw = kernel[1];
    d.oh = int32_t(oh);
    d.ow = int32_t(ow);
    d.pt = pad[0];
    d.pl = pad[2];
    d.sy = stride[0];
    d.sx = stride[1];
    return d;
}

void eval_avg_pool2d(ExecState& st, const Operator& op)
{
    const std::string OP = "AVG_POOL2D";
    if (op.attr.kind != AttrKind::Pool2d)
        throw invalid(OP, "missing attribute");
    const auto& kernel = op.attr.kernel;
    const auto& stride = op.attr.stride;
    const auto& pad = op.attr.pad;
    const DType acc_t = op.attr.acc_type;
    expect_operands(op, OP, 3, 1);
    auto input = st.get(op.inputs[0]);
    auto izp = single_value(OP, "input_zp", st.get(op.inputs[1]));
    auto ozp = single_value(OP, "output_zp", st.get(op.inputs[2]));
    const PoolDesc g = pool_geometry(OP, *input, kernel, stride, pad);
    const int64_t n = g.n, ih = g.ih, iw = g.iw, c = g.c, oh = g.oh, ow = g.ow;
    const Shape out_shape = {n, oh, ow, c};
    const DType in_t = input->dtype();
    auto declared = check_declared_output(st, OP, op.outputs[0], out_shape);
    if (declared && *declared != in_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": output dtype " + dtype_name(*declared) + " must match input dtype " +
                                            dtype_name(in_t));
    const bool supported = ((in_t == DT_INT8 || in_t == DT_INT16) && acc_t == DT_INT32) ||
                           (in_t == DT_FP16 && (acc_t == DT_FP16 || acc_t == DT_FP32)) ||
                           (in_t == DT_BF16 && acc_t == DT_FP32) || (in_t == DT_FP32 && acc_t == DT_FP32) ||
                           (is_fp8(in_t) && acc_t == DT_FP16);
    if (!supported)
        throw Error(ERR_DTYPE_MISMATCH,
                    OP + ": unsupported types input=" + dtype_name(in_t) + " acc=" + dtype_name(acc_t));
    if (izp->dtype() != in_t || ozp->dtype() != in_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": zero points must have the input dtype");
    PoolDesc d = g;
    d.xe = elem_code(in_t);
    if (dtype_is_int(in_t)) {
        const int64_t iz = int_values(*izp)[0], oz = int_values(*ozp)[0];
        if (in_t != DT_INT8 && (iz != 0 || oz != 0))
            throw invalid(OP, "zero points must be zero for non-int8 data");
        d.in_zp = iz;
        d.out_zp = oz;
        auto [lo, hi] = int_range(in_t);
        d.lo = lo;
        d.hi = hi;
    } else {
        if (float_values(*izp)[0] != 0.0 || float_values(*ozp)[0] != 0.0)
            throw invalid(OP, "zero points must be zero for floating-point data");
        d.acc_fmt = fmt_code(acc_t);
        d.out_fmt = fmt_code(in_t);
    }
    auto out = new_output(op.outputs[0], out_shape, in_t);
    void* od = out->data->device_out();
    if (shape_count(out_shape) > 0)
        kern::avg_pool2d(d, input->data->device_in(), od, st.err(), st.s());
    st.set(out);
}

// ---------------------------------------------------------------------------
// RESCALE (src/ops/type_conv.rs:111-191)
// ---------------------------------------------------------------------------
// Recipe of a deferred RESCALE from int8 to int32 (a residual operand).
struct RescaleRecipe {
    TensorPtr src;
    RescalePrep rp;
    bool consts = false;  // multiplier and shift are graph constants
};

// ---------------------------------------------------------------------------
// MAX_POOL2D (src/ops/pool.rs:233-286)
// ---------------------------------------------------------------------------
void eval_max_pool2d(ExecState& st, const Operator& op)
{
    const std::string OP = "MAX_POOL2D";
    if (op.attr.kind != AttrKind::Pool2d)
        throw invalid(OP, "missing attribute");
    expect_operands(op, OP, 1, 1);
    if (op.attr.nan_mode == NAN_UNKNOWN)
        throw invalid(OP, "nan_mode must be PROPAGATE or IGNORE");
    auto input = st.get(op.inputs[0]);
    PoolDesc d = pool_geometry(OP, *input, op.attr.kernel, op.attr.stride, op.attr.pad);
    const Shape out_shape = {d.n, d.oh, d.ow, d.c};
    const DType in_t = input->dtype();
    auto declared = check_declared_output(st, OP, op.outputs[0], out_shape);
    if (declared && *declared != in_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": output dtype " + dtype_name(*declared) + " must match input dtype " +
                                            dtype_name(in_t));
    const bool ok = in_t == DT_INT8 || in_t == DT_INT16 || in_t == DT_FP16 || in_t == DT_BF16 || in_t == DT_FP32 ||
                    is_fp8(in_t);
    if (!ok)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported dtype " + dtype_name(in_t));
    d.xe = elem_code(in_t);
    d.out_fmt = fmt_code(in_t);
    // float_lowest (src/ops/common.rs:136-140)
    const float lowest = in_t == DT_FP8E4M3 ? -448.0f : -std::numeric_limits<float>::infinity();
    auto out = new_output(op.outputs[0], out_shape, in_t);
    void* od = out->data->device_out();
    if (shape_count(out_shape) > 0)
        kern::max_pool2d(d, op.attr.nan_mode == NAN_IGNORE, lowest, input->data->device_in(), od, st.s());
    st.set(out);
}

// ---------------------------------------------------------------------------
// CAST (src/ops/type_conv.rs:14-80)
// ---------------------------------------------------------------------------
// cast_supported (:14-28): the reference model's CAST pairs.
bool cast_supported(DType from, DType to)
{
    auto is = [](DType t, std::initializer_list<DType> l) {
        for (DType u : l)
            if (u == t)
                return true;
        return false;
    };
    const auto fl16 = {DT_FP16, DT_BF16, DT_FP32};
    if (from == DT_BOOL)
        return is(to, {DT_INT8, DT_INT16, DT_INT32, DT_INT64, DT_FP32});
    if (to == DT_BOOL)
        return is(from, {DT_INT8, DT_INT16, DT_INT32, DT_INT64, DT_FP32});
    if ((from == DT_INT8 && is(to, {DT_INT16, DT_INT32})) || (from == DT_INT16 && is(to, {DT_INT8, DT_INT32})) ||
        (from == DT_INT32 && is(to, {DT_INT8, DT_INT16, DT_INT64})) || (from == DT_INT64 && to == DT_INT32))
        return true;
    if (is(from, {DT_INT8, DT_INT16, DT_INT32}) && is(to, fl16))
        return true;
    if (is(from, fl16) && is(to, {DT_INT8, DT_INT16, DT_INT32}))
        return true;
    if ((is(from, {DT_FP16, DT_BF16}) && to == DT_FP32) || (from == DT_FP32 && is(to, {DT_FP16, DT_BF16})))
        return true;
    if (is(from, fl16) && is_fp8(to))
        return true;
    if (is_fp8(from) && is(to, fl16))
        return true;
    return false;
}

// round_to (src/ops/common.rs:100-108) on the host, for the formats CAST
// converts to integers from (FP16, BF16, FP32): the saturation bounds are
// compared in the input's precision (:34-43). Round to nearest, ties to
// even; FP16 overflows to infinity from 65520.
float round_to_format(DType t, float x)
{
    if (t == DT_FP32 || !std::isfinite(x))
        return x;
    if (t == DT_BF16) {
        uint32_t u;
        std::memcpy(&u, &x, 4);
        u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
        float r;
        std::memcpy(&r, &u, 4);
        return r;
    }
    if (t != DT_FP16)
        throw Error(ERR_DTYPE_MISMATCH, std::string("round_to_format: ") + dtype_name(t));
    const float a = std::fabs(x);
    if (a >= 65520.0f)
        return std::copysign(std::numeric_limits<float>::infinity(), x);
    int e = 0;
    std::frexp(a, &e);
    const float q = std::ldexp(1.0f, std::max(e, -13) - 11);  // 11 significant bits; subnormal quantum 2^-24
    return std::nearbyint(x / q) * q;
}

void eval_cast(ExecState& st, const Operator& op)
{
    const std::string OP = "CAST";
    expect_operands(op, OP, 1, 1);
    auto input = st.get(op.inputs[0]);
    const DType from = input->dtype();
    auto declared = check_declared_output(st, OP, op.outputs[0], input->shape);
    if (!declared)
        throw invalid(OP, "output type must be declared");
    const DType to = *declared;
    if (!cast_supported(from, to))
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported cast " + dtype_name(from) + " -> " + dtype_name(to));
    CastDesc d{};
    d.from = elem_code(from);
    d.to = elem_code(to);
    d.from_float = dtype_is_int(from) || from == DT_BOOL ? 0 : 1;
    d.to_bool = to == DT_BOOL ? 1 : 0;
    d.to_float = dtype_is_int(to) || to == DT_BOOL ? 0 : 1;
    d.to_fmt = fmt_code(to);
    if (d.from_float && !d.to_float && !d.to_bool) {
        auto [lo, hi] = int_range(to);
        d.lo = lo;
        d.hi = hi;
        d.lo_bound = round_to_format(from, float(lo));
        d.hi_bound = round_to_format(from, float(hi));
    }
    auto out = new_output(op.outputs[0], input->shape, to);
    const int64_t count = shape_count(input->shape);
    void* od = out->data->device_out();
    if (count > 0)
        kern::cast(d, input->data->device_in(), count, od, st.s());
    st.set(out);
}

// ---------------------------------------------------------------------------
// CONV3D and TRANSPOSE_CONV2D (src/ops/conv.rs:505-511, :526-532): eval_conv
// (:398-500) over ConvNd with three spatial dimensions (:92-181) or the
// gather-form Transpose (:268-372), on the reference-order kernel.
// ---------------------------------------------------------------------------
void eval_conv_nd(ExecState& st, const Operator& op, bool transpose)
{
    const std::string OP = transpose ? "TRANSPOSE_CONV2D" : "CONV3D";
    if (op.attr.kind != (transpose ? AttrKind::TransposeConv2d : AttrKind::Conv3d))
        throw invalid(OP, "missing attribute");
    expect_operands(op, OP, 5, 1);
    auto input = st.get(op.inputs[0]);
    auto weight = st.get(op.inputs[1]);
    auto bias = st.get(op.inputs[2]);
    auto in_zp = single_value(OP, "input_zp", st.get(op.inputs[3]));
    auto w_zp = single_value(OP, "weight_zp", st.get(op.inputs[4]));
    expect_rank(OP, "bias", *bias, 1);
    DirectConvDesc d{};
    d.m = 1;
    d.dy = d.dx = 1;
    Shape out_shape;
    if (transpose) {
        // Transpose::new (:284-330)
        expect_rank(OP, "input", *input, 4);
        expect_rank(OP, "weight", *weight, 4);
        const auto& out_pad = op.attr.out_pad;
        const auto& stride = op.attr.stride;
        if (out_pad.size() != 4 || stride.size() != 2)
            throw invalid(OP, "out_pad must have 4 elements and stride 2");
        for (int32_t sv : stride)
            if (sv < 1)
                throw invalid(OP, "stride must be at least 1");
        const int64_t n = input->shape[0], ih = input->shape[1], iw = input->shape[2], ic = input->shape[3];
        const int64_t oc = weight->shape[0], kh = weight->shape[1], kw = weight->shape[2];
        if (weight->shape[3] != ic)
            throw Error(ERR_SHAPE_MISMATCH, OP + ": weight input channels " + std::to_string(weight->shape[3]) +
                                                " != input channels " + std::to_string(ic));
        for (size_t i = 0; i < 4; i++)
            if (int64_t(out_pad[i]) <= -(i < 2 ? kh : kw))
                throw invalid(OP, "out_pad must be greater than -kernel size");
        const int64_t oh = (ih - 1) * stride[0] + out_pad[0] + out_pad[1] + kh;
        const int64_t ow = (iw - 1) * stride[1] + out_pad[2] + out_pad[3] + kw;
        if (oh < 1 || ow < 1)
            throw invalid(OP, "output size " + std::to_string(oh) + "x" + std::to_string(ow) + " must be positive");
        d.transpose = 1;
        d.n = int32_t(n);
        d.ih = int32_t(ih);
        d.iw = int32_t(iw);
        d.c = int32_t(ic);
        d.oc = int32_t(oc);
        d.kh = int32_t(kh);
        d.kw = int32_t(kw);
        d.oh = int32_t(oh);
        d.ow = int32_t(ow);
        d.pt = out_pad[0];
        d.pl = out_pad[2];
        d.sy = stride[0];
        d.sx = stride[1];
        out_shape = {n, oh, ow, oc};
    } else {
        // ConvNd::new with three dimensions (:106-139)
        expect_rank(OP, "input", *input, 5);
        expect_rank(OP, "weight", *weight, 5);
        const auto& pad = op.attr.pad;
        const auto& stride = op.attr.stride;
        const auto& dil = op.attr.dilation;
        if (pad.size() != 6 || stride.size() != 3 || dil.size() != 3)
            throw invalid(OP, "pad must have 6 elements, stride and dilation 3");
        for (int32_t p : pad)
            if (p < 0)
                throw invalid(OP, "pad must be non-negative");
        for (int32_t sv : stride)
            if (sv < 1)
                throw invalid(OP, "stride must be at least 1");
        for (int32_t dv : dil)
            if (dv < 1)
                throw invalid(OP, "dilation must be at least 1");
        const int64_t ic = input->shape[4];
        if (weight->shape[4] != ic)
            throw Error(ERR_SHAPE_MISMATCH, OP + ": weight input channels " + std::to_string(weight->shape[4]) +
                                                " != input channels " + std::to_string(ic));
        const int64_t od = output_extent(OP, input->shape[1], pad[0], pad[1], weight->shape[1], dil[0], stride[0]);
        const int64_t oh = output_extent(OP, input->shape[2], pad[2], pad[3], weight->shape[2], dil[1], stride[1]);
        const int64_t ow = output_extent(OP, input->shape[3], pad[4], pad[5], weight->shape[3], dil[2], stride[2]);
        d.n = int32_t(input->shape[0]);
        d.id = int32_t(input->shape[1]);
        d.ih = int32_t(input->shape[2]);
        d.iw = int32_t(input->shape[3]);
        d.c = int32_t(ic);
        d.oc = int32_t(weight->shape[0]);
        d.kd = int32_t(weight->shape[1]);
        d.kh = int32_t(weight->shape[2]);
        d.kw = int32_t(weight->shape[3]);
        d.od = int32_t(od);
        d.oh = int32_t(oh);
        d.ow = int32_t(ow);
        d.pf = pad[0];
        d.pt = pad[2];
        d.pl = pad[4];
        d.sz = stride[0];
        d.sy = stride[1];
        d.sx = stride[2];
        d.dz = dil[0];
        d.dy = dil[1];
        d.dx = dil[2];
        out_shape = {input->shape[0], od, oh, ow, weight->shape[0]};
    }
    const int64_t oc = out_shape.back();
    const int64_t bc = bias->shape[0];
    if (bc != oc && bc != 1)
        throw Error(ERR_SHAPE_MISMATCH, OP + ": bias channels " + std::to_string(bc) +
                                            " must be 1 or match output channels " + std::to_string(oc));
    const DType in_t = input->dtype(), w_t = weight->dtype(), out_t = bias->dtype(), acc_t = op.attr.acc_type;
    auto declared = check_declared_output(st, OP, op.outputs[0], out_shape);
    if (declared && *declared != out_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": output dtype " + dtype_name(*declared) + " does not match bias dtype " +
                                            dtype_name(out_t));
    if (!standard_types(in_t, w_t, acc_t, out_t))
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported types input=" + dtype_name(in_t) + " weight=" +
                                            dtype_name(w_t) + " acc=" + dtype_name(acc_t) + " output=" +
                                            dtype_name(out_t));
    if (in_zp->dtype() != in_t || w_zp->dtype() != w_t)
        throw Error(ERR_DTYPE_MISMATCH, OP + ": zero points must match input/weight dtypes");
    const bool is_int = dtype_is_int(acc_t);
    if (is_int) {
        d.zp_x = int_values(*in_zp)[0];
        d.zp_w = int_values(*w_zp)[0];
        if (d.zp_x != 0 && in_t != DT_INT8)
            throw invalid(OP, "input zero point must be zero for non-int8 input");
        if (d.zp_w != 0 && w_t != DT_INT8)
            throw invalid(OP, "weight zero point must be zero for non-int8 weight");
    } else {
        d.fzp_x = float(float_values(*in_zp)[0]);
        d.fzp_w = float(float_values(*w_zp)[0]);
        if (d.fzp_x != 0.0f || d.fzp_w != 0.0f)
            throw invalid(OP, "zero points must be zero for floating-point operands");
    }
    const int64_t count = shape_count(out_shape);
    if (shape_count(input->shape) >= (int64_t(1) << 31) || count >= (int64_t(1) << 31))
        throw Error(ERR_SHAPE_MISMATCH, OP + ": tensors of 2^31 elements or more are not supported");
    d.xe = elem_code(in_t);
    d.we = elem_code(w_t);
    d.be = elem_code(out_t);
    d.oe = elem_code(out_t);
    d.acc = is_int ? (acc_t == DT_INT32 ? ACC_I32 : ACC_I64) : float_acc(acc_t);
    d.bias_len = int32_t(bc);
    d.out_fmt = fmt_code(out_t);
    auto out = new_output(op.outputs[0], out_shape, out_t);
    void* od = out->data->device_out();
    if (count > 0)
        kern::direct_conv(d, input->data->device_in(), weight->data->device_in(), bias->data->device_in(), od, st.s());
    st.set(out);
}

void eval_rescale(ExecState& st, const Operator& op, size_t index)
{
    const std::string OP = "RESCALE";
    if (op.attr.kind != AttrKind::Rescale)
        throw invalid(OP, "missing attribute");
    expect_operands(op, OP, 5, 1);
    auto input = st.get(op.inputs[0]);
    auto mult = st.get(op.inputs[1]);
    auto shift = st.get(op.inputs[2]);
    auto izp = st.get(op.inputs[3]);
    auto ozp = st.get(op.inputs[4]);
    auto pend = st.pending.find(op.outputs[0]);
    if (pend != st.pending.end()) {
        // Produced by the fused kernel of the operator feeding this one; the
        // same checks passed when that kernel was planned.
        st.set(pend->second);
        st.pending.erase(pend);
        return;
    }
    RescalePrep p = prepare_rescale(st, op, *input, mult, shift, izp, ozp);
    const int64_t count = shape_count(p.shape);
    if (st.opts.fusion && st.plan && st.plan->residual_input[index] && p.in_t == DT_INT8 && p.out_t == DT_INT32) {
        auto src = input;
        auto out = virtual_output(op.outputs[0], p.shape, p.out_t, [src, p](Storage& o) {
            Stream& s = thread_stream();
            const void* x = src->data->device_in();
            kern::rescale(p.rs, E_I8, x, o.count, o.device_out(), s.err, s.s);
        });
        auto recipe = std::make_shared<RescaleRecipe>();
        recipe->src = input;
        recipe->rp = p;
        recipe->consts = st.is_const(op.inputs[1]) && st.is_const(op.inputs[2]);
        // The recipe rides on the virtual storage as an opaque aux entry.
        out->data->aux = std::shared_ptr<Storage>(recipe, reinterpret_cast<Storage*>(recipe.get()));
        out->data->aux_kind = 100;
        st.set(out);
        return;
    }
    auto out = new_output(op.outputs[0], p.shape, p.out_t);
    void* od = out->data->device_out();
    if (count > 0)
        kern::rescale(p.rs, elem_code(p.in_t), input->data->device_in(), count, od, st.err(), st.s());
    st.set(out);
}

// ---------------------------------------------------------------------------
// CLAMP (src/ops/elementwise.rs:314-343)
// ---------------------------------------------------------------------------
void eval_clamp(ExecState& st, const Operator& op)
{
    const std::string OP = "CLAMP";
    if (op.attr.kind != AttrKind::Clamp)
        throw invalid(OP, "missing attribute");
    if (op.attr.nan_mode == NAN_UNKNOWN)
        throw invalid(OP, "nan_mode must be PROPAGATE or IGNORE");
    const DType t = st.get(op.inputs.empty() ? std::string() : op.inputs[0])->dtype();
    StoragePtr mn, mx;
    try {
        mn = storage_from_raw_bytes(t, op.attr.min_val.data(), op.attr.min_val.size(), 1);
        mx = storage_from_raw_bytes(t, op.attr.max_val.data(), op.attr.max_val.size(), 1);
    } catch (const Error&) {
        throw invalid(OP, "malformed min/max");
    }
    expect_operands(op, OP, 1, 1);
    auto input = st.get(op.inputs[0]);
    if (!(t == DT_FP16 || t == DT_BF16 || t == DT_FP32 || t == DT_INT8 || t == DT_INT16))
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported dtype " + dtype_name(t));
    Tensor tmn, tmx;
    tmn.data = mn;
    tmx.data = mx;
    int64_t ilo = 0, ihi = 0;
    float flo = 0, fhi = 0;
    if (dtype_is_int(t)) {
        ilo = int_values(tmn)[0];
        ihi = int_values(tmx)[0];
        if (ihi < ilo)
            throw invalid(OP, "max_val must not be smaller than min_val");
    } else {
        flo = float(float_values(tmn)[0]);
        fhi = float(float_values(tmx)[0]);
        if (std::isnan(flo) || std::isnan(fhi) || fhi < flo)
            throw invalid(OP, "min_val/max_val must be ordered and not NaN");
    }
    check_finish(st, OP, op.outputs[0], input->shape, t);
    auto pend = st.pending.find(op.outputs[0]);
    if (pend != st.pending.end()) {
        st.set(pend->second);
        st.pending.erase(pend);
        return;
    }
    auto out = new_output(op.outputs[0], input->shape, t);
    void* od = out->data->device_out();
    const int64_t count = shape_count(input->shape);
    if (count > 0)
        kern::clamp(elem_code(t), input->data->device_in(), count, ilo, ihi, flo, fhi,
                    op.attr.nan_mode == NAN_IGNORE, od, st.s());
    st.set(out);
}

// ---------------------------------------------------------------------------
// ADD (src/ops/elementwise.rs:57-107, :359-397)
// ---------------------------------------------------------------------------
void eval_add(ExecState& st, const Operator& op, size_t index)
{
    const std::string OP = "ADD";
    expect_operands(op, OP, 2, 1);
    auto a = st.get(op.inputs[0]);
    auto b = st.get(op.inputs[1]);
    if (a->dtype() != b->dtype())
        throw Error(ERR_DTYPE_MISMATCH, OP + ": input dtypes " + dtype_name(a->dtype()) + " and " +
                                            dtype_name(b->dtype()) + " differ");
    const size_t rank = a->shape.size();
    if (b->shape.size() != rank)
        throw Error(ERR_SHAPE_MISMATCH, OP + ": operand ranks differ");
    Shape out(rank);
    for (size_t d = 0; d < rank; d++) {
        int64_t dim = 1;
        for (int64_t s : {a->shape[d], b->shape[d]}) {
            if (s != 1) {
                if (dim != 1 && dim != s)
                    throw Error(ERR_BROADCAST, OP + ": shapes " + shape_str(a->shape) + " and " + shape_str(b->shape) +
                                                   " are not broadcastable");
                dim = s;
            }
        }
        out[d] = dim;
    }
    const DType t = a->dtype();
    if (!(t == DT_FP16 || t == DT_BF16 || t == DT_FP32 || t == DT_INT32 || t == DT_INT64))
        throw Error(ERR_DTYPE_MISMATCH, OP + ": unsupported dtype " + dtype_name(t));
    check_finish(st, OP, op.outputs[0], out, t);
    if (rank > 6)
        throw Error(ERR_SHAPE_MISMATCH, OP + ": rank above 6");
    const int64_t count = shape_count(out);

    // Quantised residual: ADD(RESCALE(int8), RESCALE(int8)) -> RESCALE(int8).
    auto recipe_of = [](const TensorPtr& x) -> RescaleRecipe* {
        if (x->data->is_virtual() && x->data->aux_kind == 100)
            return reinterpret_cast<RescaleRecipe*>(x->data->aux.get());
        return nullptr;
    };
    if (st.opts.fusion && st.plan && st.plan->residual_tail[index] >= 0 && t == DT_INT32 && a->shape == out &&
        b->shape == out && !out.empty()) {
        RescaleRecipe* ra = recipe_of(a);
        RescaleRecipe* rb = recipe_of(b);
        if (ra && rb) {
            const Operator& rop = st.block->operators[st.plan->residual_tail[index]];
            TensorPtr ops[4];
            bool ok = rop.attr.kind == AttrKind::Rescale && rop.inputs.size() == 5 && rop.outputs.size() == 1;
            for (int i = 0; ok && i < 4; i++)
                ok = (ops[i] = st.resolve(rop.inputs[1 + i])) != nullptr;
            std::optional<RescalePrep> tail;
            if (ok) {
                Tensor tmp;
                tmp.shape = out;
                tmp.data = std::make_shared<Storage>();
                tmp.data->dtype = DT_INT32;
                tmp.data->count = count;
                try {
                    tail = prepare_rescale(st, rop, tmp, ops[0], ops[1], ops[2], ops[3]);
                } catch (const Error&) {
                    tail.reset();
                }
            }
            if (tail && tail->out_t == DT_INT8) {
                auto fin = new_output(rop.outputs[0], out, DT_INT8);
                void* fo = fin->data->device_out();
                // A held-back convolution as either operand's source takes
                // the residual into its epilogue; otherwise the residual
                // kernel reads both int8 sources.
                auto conv_of = [](const TensorPtr& x) -> ConvResRecipe* {
                    if (x->data->is_virtual() && x->data->aux_kind == AUX_CONV_RES)
                        return reinterpret_cast<ConvResRecipe*>(x->data->aux.get());
                    return nullptr;
                };
                const bool cacheable =
                    ra->consts && rb->consts && st.is_const(rop.inputs[1]) && st.is_const(rop.inputs[2]);
                bool done = false;
                for (int side = 0; side < 2 && !done; side++) {
                    RescaleRecipe* ry = side == 0 ? ra : rb;
                    RescaleRecipe* rx = side == 0 ? rb : ra;
                    ConvResRecipe* cr = conv_of(ry->src);
                    if (cr && !conv_of(rx->src))
                        done = cr->launch(fo, ry->rp.rs, rx->rp.rs, tail->rs, cacheable,
                                          static_cast<const int8_t*>(rx->src->data->device_in()), st.err(), st.s());
                }
                if (!done)
                    kern::residual_add_i8(ra->rp.rs, rb->rp.rs, tail->rs,
                                          static_cast<const int8_t*>(ra->src->data->device_in()),
                                          static_cast<const int8_t*>(rb->src->data->device_in()), count, out.back(),
                                          fo, st.err(), st.s());
                BroadcastDesc bd{};
                bd.rank = int32_t(rank);
                int64_t s = 1;
                for (int d = int(rank) - 1; d >= 0; d--) {
                    bd.out_dims[d] = out[d];
                    bd.a_strides[d] = s;
                    bd.b_strides[d] = s;
                    s *= out[d];
                }
                auto keep = tail->params;
                auto sum = virtual_output(op.outputs[0], out, DT_INT32, [a, b, bd, keep](Storage& o) {
                    Stream& s = thread_stream();
                    const void* ad = a->data->device_in();
                    const void* bdp = b->data->device_in();
                    kern::add(E_I32, bd, ad, bdp, o.device_out(), o.count, s.s);
                });
                st.set(sum);
                st.pending[rop.outputs[0]] = fin;
                return;
            }
        }
    }

    BroadcastDesc bd{};
    bd.rank = int32_t(rank);
    int64_t sa = 1, sb = 1;
    for (int d = int(rank) - 1; d >= 0; d--) {
        bd.out_dims[d] = out[d];
        bd.a_strides[d] = a->shape[d] == 1 ? 0 : sa;
        bd.b_strides[d] = b->shape[d] == 1 ? 0 : sb;
        sa *= a->shape[d];
        sb *= b->shape[d];
    }
    auto o = new_output(op.outputs[0], out, t);
    void* od = o->data->device_out();
    if (count > 0)
        kern::add(elem_code(t), bd, a->data->device_in(), b->data->device_in(), od, count, st.s());
    st.set(o);
}

}  // namespace

void dispatch(ExecState& st, const Operator& op, size_t index)
{
    switch (op.op) {
    case OP_CONST:
    case OP_CONST_SHAPE: eval_const(st, op); return;
    case OP_IDENTITY: eval_identity(st, op); return;
    case OP_RESHAPE: eval_reshape(st, op); return;
    case OP_TRANSPOSE: eval_transpose(st, op); return;
    case OP_CONV2D: eval_conv(st, op, index, false); return;
    case OP_DEPTHWISE_CONV2D: eval_conv(st, op, index, true); return;
    case OP_MATMUL: eval_matmul(st, op, index, false); return;
    case OP_MATMUL_T: eval_matmul(st, op, index, true); return;
    case OP_CONV3D: eval_conv_nd(st, op, false); return;
    case OP_TRANSPOSE_CONV2D: eval_conv_nd(st, op, true); return;
    case OP_AVG_POOL2D: eval_avg_pool2d(st, op); return;
    case OP_MAX_POOL2D: eval_max_pool2d(st, op); return;
    case OP_CAST: eval_cast(st, op); return;
    case OP_RESCALE: eval_rescale(st, op, index); return;
    case OP_CLAMP: eval_clamp(st, op); return;
    case OP_ADD: eval_add(st, op, index); return;
    default: break;
    }
    if (op.op > OP_LAST)
        throw Error(ERR_UNSUPPORTED_OP, "op code " + std::to_string(op.op));
    throw Error(ERR_UNSUPPORTED_OP, std::string(op_name(op.op)) + " (not part of the MI355X execution path)");
}

}  // namespace tosa
