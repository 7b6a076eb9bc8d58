// Dataflow execution of one basic block, after src/interpreter.rs:154-253.
//
// The reference keeps a FIFO ready queue seeded with every ready operator in
// graph order (CONST is always ready), and after each operator rescans the
// whole block, appending newly ready operators in graph order. Here the same
// order is produced in O(edges): each operator keeps a count of distinct
// input names still missing, and an operator's outputs release exactly the
// consumers whose count drops to zero, appended in graph order. Hooks see
// the same call sequence as in the reference: pre_op, on_tensor_alloc per
// output, post_op, with on_tensor_free never called.
//
// Kernels are launched asynchronously on the thread's stream; the run ends
// with one stream synchronisation and one read of the device error word.
#include "interpreter.h"

#include <algorithm>
#include <cstdlib>
#include <deque>

namespace tosa {

RunOptions& default_run_options()
{
    static RunOptions opts = [] {
        RunOptions o;
        if (const char* f = std::getenv("TOSA_MI355X_FUSION"))
            o.fusion = std::atoi(f) != 0;
        if (const char* s = std::getenv("TOSA_MI355X_STRICT_FLOAT"))
            o.strict_float = std::atoi(s) != 0;
        if (const char* d = std::getenv("TOSA_MI355X_DEFERRED"))
            o.deferred = std::atoi(d) != 0;
        return o;
    }();
    return opts;
}

// ---------------------------------------------------------------------------
// Fusion plan
// ---------------------------------------------------------------------------
FusionPlan FusionPlan::build(const BasicBlock& b)
{
    const size_t n = b.operators.size();
    FusionPlan p;
    p.rescale_after.assign(n, -1);
    p.clamp_after.assign(n, -1);
    p.residual_tail.assign(n, -1);
    p.residual_input.assign(n, false);
    p.residual_head.assign(n, false);

    std::unordered_map<std::string, std::vector<int>> consumers;  // name -> consuming ops (one entry per use)
    std::unordered_map<std::string, int> producers;
    std::unordered_map<std::string, int> produced_count;
    for (size_t i = 0; i < n; i++) {
        for (const auto& in : b.operators[i].inputs)
            consumers[in].push_back(int(i));
        for (const auto& out : b.operators[i].outputs) {
            producers[out] = int(i);
            produced_count[out]++;
        }
    }
    std::unordered_set<std::string> block_out(b.outputs.begin(), b.outputs.end());
    // A tensor that only `op` reads, once, as its first operand; produced by
    // exactly one operator and not a block output.
    auto sole_first_use = [&](const std::string& name, uint32_t opcode) -> int {
        if (block_out.count(name) || produced_count[name] != 1)
            return -1;
        auto it = consumers.find(name);
        if (it == consumers.end() || it->second.size() != 1)
            return -1;
        const int c = it->second[0];
        const Operator& co = b.operators[c];
        if (co.op != opcode || co.inputs.empty() || co.inputs[0] != name)
            return -1;
        return c;
    };
    for (size_t i = 0; i < n; i++) {
        const Operator& o = b.operators[i];
        if ((o.op == OP_CONV2D || o.op == OP_DEPTHWISE_CONV2D || o.op == OP_MATMUL || o.op == OP_MATMUL_T) &&
            o.outputs.size() == 1) {
            const int j = sole_first_use(o.outputs[0], OP_RESCALE);
            if (j >= 0) {
                p.rescale_after[i] = j;
                const Operator& r = b.operators[j];
                if (r.outputs.size() == 1)
                    p.clamp_after[j] = sole_first_use(r.outputs[0], OP_CLAMP);
            }
        }
        if (o.op == OP_ADD && o.inputs.size() == 2 && o.outputs.size() == 1 && o.inputs[0] != o.inputs[1]) {
            bool ok = true;
            int ins[2];
            for (int k = 0; k < 2 && ok; k++) {
                const std::string& name = o.inputs[k];
                auto it = consumers.find(name);
                auto pr = producers.find(name);
                ok = !block_out.count(name) && produced_count[name] == 1 && it != consumers.end() &&
                     it->second.size() == 1 && pr != producers.end() && b.operators[pr->second].op == OP_RESCALE;
                if (ok)
                    ins[k] = pr->second;
            }
            const int tail = ok ? sole_first_use(o.outputs[0], OP_RESCALE) : -1;
            if (tail >= 0 && ins[0] != ins[1]) {
                p.residual_tail[i] = tail;
                p.residual_input[ins[0]] = true;
                p.residual_input[ins[1]] = true;
            }
        }
    }
    // A convolution whose fused RESCALE result (no CLAMP after it) is read
    // only by a residual RESCALE.
    for (size_t i = 0; i < n; i++) {
        const int j = p.rescale_after[i];
        if (b.operators[i].op != OP_CONV2D || j < 0 || p.clamp_after[j] >= 0 || b.operators[j].outputs.size() != 1)
            continue;
        const int k = sole_first_use(b.operators[j].outputs[0], OP_RESCALE);
        if (k >= 0 && p.residual_input[k])
            p.residual_head[i] = true;
    }
    return p;
}

// ---------------------------------------------------------------------------
// Interpreter
// ---------------------------------------------------------------------------
BlockIndex BlockIndex::build(const BasicBlock& b)
{
    BlockIndex x;
    for (const auto& td : b.tensors)
        x.defs[td.name] = &td;
    for (const auto& o : b.operators)
        if ((o.op == OP_CONST || o.op == OP_CONST_SHAPE) && !o.outputs.empty()) {
            auto it = x.defs.find(o.outputs[0]);
            if (it != x.defs.end())
                x.const_defs[o.outputs[0]] = it->second;
        }
    // Rank check (src/interpreter.rs:157-163): the first offending tensor.
    for (const auto& t : b.tensors)
        if (t.dtype != DT_SHAPE && t.shape.size() > MAX_RANK) {
            x.rank_error = "tensor '" + t.name + "' has rank " + std::to_string(t.shape.size()) +
                           ", above the maximum of " + std::to_string(MAX_RANK);
            break;
        }
    auto id_of = [&x](const std::string& name) {
        auto it = x.ids.emplace(name, int(x.ids.size())).first;
        return it->second;
    };
    const size_t n = b.operators.size();
    x.op_inputs.resize(n);
    x.op_outputs.resize(n);
    for (size_t i = 0; i < n; i++) {
        const Operator& o = b.operators[i];
        if (o.op != OP_CONST) {
            for (const auto& name : o.inputs)
                x.op_inputs[i].push_back(id_of(name));
            std::sort(x.op_inputs[i].begin(), x.op_inputs[i].end());
            x.op_inputs[i].erase(std::unique(x.op_inputs[i].begin(), x.op_inputs[i].end()), x.op_inputs[i].end());
        }
        for (const auto& name : o.outputs)
            x.op_outputs[i].push_back(id_of(name));
    }
    return x;
}

Interpreter::Interpreter(Graph graph)
    : graph_(std::move(graph)), consts_(new ConstCache()), sched_(new ScheduleCache())
{
    if (const BasicBlock* b = graph_.main_block()) {
        plan_ = FusionPlan::build(*b);
        index_ = BlockIndex::build(*b);
    }
}

// The schedule for this run's input names: the last one built when the names
// are the same (the usual case of repeated runs), else a new one.
std::shared_ptr<const Schedule> Interpreter::schedule_for(const TensorMap& inputs) const
{
    {
        std::lock_guard<std::mutex> lk(sched_->mu);
        const auto& last = sched_->last;
        if (last && last->input_names.size() == inputs.size()) {
            bool same = true;
            for (const auto& kv : inputs)
                if (!last->input_names.count(kv.first)) {
                    same = false;
                    break;
                }
            if (same)
                return last;
        }
    }
    auto s = std::make_shared<Schedule>();
    const size_t n = index_.op_inputs.size();
    s->available.assign(index_.ids.size(), 0);
    for (const auto& kv : inputs) {
        s->input_names.insert(kv.first);
        auto it = index_.ids.find(kv.first);
        if (it != index_.ids.end())
            s->available[it->second] = 1;
    }
    s->missing.assign(n, 0);
    s->waiting.resize(index_.ids.size());
    for (size_t i = 0; i < n; i++)
        for (int id : index_.op_inputs[i])
            if (!s->available[id]) {
                s->missing[i]++;
                s->waiting[id].push_back(i);
            }
    for (size_t i = 0; i < n; i++)
        if (s->missing[i] == 0)
            s->queue.push_back(i);
    std::lock_guard<std::mutex> lk(sched_->mu);
    sched_->last = s;
    return s;
}

Interpreter Interpreter::from_flatbuffer(const uint8_t* data, size_t len)
{
    return Interpreter(Graph::from_flatbuffer(data, len));
}

TensorMap Interpreter::run(const TensorMap& inputs, InterpreterHook& hook) const
{
    return run(inputs, hook, default_run_options());
}

TensorMap Interpreter::run(const TensorMap& inputs, InterpreterHook& hook, const RunOptions& opts) const
{
    const BasicBlock* block = graph_.main_block();
    if (!block)
        throw Error(ERR_GRAPH, "no main block found");

    ExecState st;
    st.block = block;
    st.defs = &index_.defs;
    st.const_defs = &index_.const_defs;
    st.tensors = inputs;
    st.consts = consts_.get();
    st.plan = &plan_;
    st.opts = opts;
    if (hook.reads_data())
        st.opts.fusion = false;  // every intermediate is materialised for such a hook

    if (!index_.rank_error.empty())
        throw Error(ERR_SHAPE_MISMATCH, index_.rank_error);

    const auto& ops = block->operators;
    const size_t n = ops.size();
    // Count of distinct input names each operator still misses, and the
    // consumers of each name (the part that depends only on the graph and the
    // input names is built once and copied here).
    const std::shared_ptr<const Schedule> sched = schedule_for(inputs);
    std::vector<char> available = sched->available;
    std::vector<size_t> missing = sched->missing;
    std::vector<bool> executed(n, false), queued(n, false);
    std::deque<size_t> queue(sched->queue.begin(), sched->queue.end());
    for (size_t i : sched->queue)
        queued[i] = true;

    const bool sync_each = !hook.is_noop() && hook.needs_sync();
    const bool noop = hook.is_noop();

    size_t ops_executed = 0;
    while (!queue.empty()) {
        const size_t idx = queue.front();
        queue.pop_front();
        queued[idx] = false;
        if (executed[idx])
            continue;
        const Operator& op = ops[idx];
        const OpInfo info{op.op, idx};
        TensorRefs in_refs;
        if (!noop) {
            for (const auto& name : op.inputs) {
                auto it = st.tensors.find(name);
                if (it != st.tensors.end())
                    in_refs.push_back(it->second.get());
            }
            hook.pre_op(info, in_refs);
        }
        dispatch(st, op, idx);
        if (!noop) {
            if (sync_each && st.has_stream()) {
                if (uint32_t e = read_error_word(st.stream()))
                    throw Error(ERR_GRAPH, std::string(op_name(op.op)) + ": " + device_error_message(e));
            }
            TensorRefs out_refs;
            for (const auto& name : op.outputs) {
                auto it = st.tensors.find(name);
                if (it != st.tensors.end())
                    out_refs.push_back(it->second.get());
            }
            for (const Tensor* t : out_refs)
                hook.on_tensor_alloc(t->name, t->shape, t->dtype(), t->size_bytes());
            in_refs.clear();
            for (const auto& name : op.inputs) {
                auto it = st.tensors.find(name);
                if (it != st.tensors.end())
                    in_refs.push_back(it->second.get());
            }
            hook.post_op(info, in_refs, out_refs);
        }
        executed[idx] = true;
        ops_executed++;
        // Newly available outputs release waiting operators, in graph order.
        std::vector<size_t> ready;
        for (int id : index_.op_outputs[idx]) {
            if (available[id])
                continue;
            available[id] = 1;
            for (size_t j : sched->waiting[id])
                if (--missing[j] == 0 && !executed[j] && !queued[j])
                    ready.push_back(j);
        }
        std::sort(ready.begin(), ready.end());
        for (size_t j : ready) {
            queue.push_back(j);
            queued[j] = true;
        }
    }

    if (ops_executed < n) {
        std::string names = "[";
        bool first = true;
        for (size_t i = 0; i < n; i++)
            if (!executed[i]) {
                names += std::string(first ? "" : ", ") + "\"" + op_name(ops[i].op) + "\"";
                first = false;
            }
        throw Error(ERR_GRAPH, "could not execute all ops, stuck on: " + names + "]");
    }

    TensorMap outputs;
    for (const auto& name : block->outputs) {
        auto it = st.tensors.find(name);
        if (it == st.tensors.end())
            continue;
        TensorPtr t = it->second;
        st.tensors.erase(it);
        if (t->data && t->data->is_virtual()) {
            st.stream();
            t->data->device_in();
        }
        outputs.emplace(name, t);
    }
    if (st.has_stream() && !st.opts.deferred) {
        if (uint32_t e = read_error_word(st.stream()))
            throw Error(ERR_GRAPH, device_error_message(e));
    }
    return outputs;
}

TensorMap run_graph(const uint8_t* data, size_t len, const TensorMap& inputs)
{
    Interpreter interp = Interpreter::from_flatbuffer(data, len);
    NoopHook hook;
    return interp.run(inputs, hook);
}

TensorMap run_graph_with_stats(const uint8_t* data, size_t len, const TensorMap& inputs, StatsCollector& stats)
{
    Interpreter interp = Interpreter::from_flatbuffer(data, len);
    return interp.run(inputs, stats);
}

TensorMap run_graph_with_hooks(const uint8_t* data, size_t len, const TensorMap& inputs, InterpreterHook& hooks)
{
    Interpreter interp = Interpreter::from_flatbuffer(data, len);
    return interp.run(inputs, hooks);
}

}  // namespace tosa
