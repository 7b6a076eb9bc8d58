#include "hooks.h"

#include <cstdio>

namespace tosa {

void HookSet::pre_op(const OpInfo& o, const TensorRefs& in)
{
    for (auto& h : hooks_)
        h->pre_op(o, in);
}
void HookSet::post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out)
{
    for (auto& h : hooks_)
        h->post_op(o, in, out);
}
void HookSet::on_tensor_alloc(const std::string& n, const Shape& s, DType t, size_t b)
{
    for (auto& h : hooks_)
        h->on_tensor_alloc(n, s, t, b);
}
void HookSet::on_tensor_free(const std::string& n, size_t b)
{
    for (auto& h : hooks_)
        h->on_tensor_free(n, b);
}
bool HookSet::needs_sync() const
{
    for (auto& h : hooks_)
        if (h->needs_sync())
            return true;
    return false;
}
bool HookSet::reads_data() const
{
    for (auto& h : hooks_)
        if (h->reads_data())
            return true;
    return false;
}

std::string StatsCollector::summary() const
{
    std::string s = "Total ops executed: " + std::to_string(total_ops_executed) + "\n";
    s += "Peak memory: " + std::to_string(peak_memory_bytes) + " bytes\n";
    for (const auto& [name, st] : op_stats) {  // std::map: sorted by name
        char line[256];
        std::snprintf(line, sizeof(line), "\n  %-16s count=%-6llu time=%8.3fms  elements_in=%-10llu elements_out=%-10llu",
                      name.c_str(), (unsigned long long)st.count, st.total_time * 1000.0,
                      (unsigned long long)st.total_input_elements, (unsigned long long)st.total_output_elements);
        s += line;
    }
    return s;
}

void StatsCollector::pre_op(const OpInfo&, const TensorRefs&)
{
    started_ = true;
    start_ = std::chrono::steady_clock::now();
}

void StatsCollector::post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out)
{
    double elapsed = 0;
    if (started_)
        elapsed = std::chrono::duration<double>(std::chrono::steady_clock::now() - start_).count();
    OpStats& e = op_stats[op_name(o.op)];
    e.count++;
    e.total_time += elapsed;
    for (const Tensor* t : in)
        e.total_input_elements += uint64_t(t->element_count());
    for (const Tensor* t : out)
        e.total_output_elements += uint64_t(t->element_count());
    total_ops_executed++;
}

void StatsCollector::on_tensor_alloc(const std::string&, const Shape&, DType, size_t bytes)
{
    current_memory_bytes += bytes;
    if (current_memory_bytes > peak_memory_bytes)
        peak_memory_bytes = current_memory_bytes;
}

void StatsCollector::on_tensor_free(const std::string&, size_t bytes)
{
    current_memory_bytes = bytes > current_memory_bytes ? 0 : current_memory_bytes - bytes;
}

static uint64_t estimate_flops(uint32_t op, const TensorRefs& in, const TensorRefs& out)
{
    auto first_count = [&]() -> uint64_t { return out.empty() ? 0 : uint64_t(out[0]->element_count()); };
    switch (op) {
    case OP_ADD:
    case OP_SUB:
    case OP_MUL:
    case 32 /* ABS */:
    case 41 /* NEGATE */:
    case 26 /* MAXIMUM */:
    case 27 /* MINIMUM */: return first_count();
    case 37 /* EXP */:
    case 39 /* LOG */:
    case 44 /* SIN */:
    case 36 /* COS */:
    case 14 /* TANH */:
    case 13 /* SIGMOID */:
    case 12 /* ERF */:
    case 43 /* RSQRT */:
    case 42 /* RECIPROCAL */:
    case 29 /* POW */: return first_count() * 10;
    case OP_MATMUL:
        if (in.size() >= 2 && in[0]->shape.size() == 3) {
            const uint64_t n = in[0]->shape[0], h = in[0]->shape[1], c = in[0]->shape[2], w = in[1]->shape[2];
            return 2 * n * h * w * c;
        }
        return 0;
    case OP_CONV2D:
        if (in.size() >= 2 && !out.empty() && out[0]->shape.size() == 4 && in[1]->shape.size() == 4) {
            const auto& o = out[0]->shape;
            const auto& w = in[1]->shape;
            return 2ull * o[0] * o[1] * o[2] * o[3] * w[1] * w[2] * w[3];
        }
        return 0;
    default: return 0;
    }
}

void FlopCounter::post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out)
{
    const uint64_t f = estimate_flops(o.op, in, out);
    total_flops += f;
    flops_by_op[op_name(o.op)] += f;
}

void OpTrace::post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out)
{
    TraceEntry e;
    e.op = op_name(o.op);
    e.op_index = o.op_index;
    for (const Tensor* t : in)
        e.input_shapes.push_back(t->shape);
    for (const Tensor* t : out)
        e.output_shapes.push_back(t->shape);
    entries.push_back(std::move(e));
}

}  // namespace tosa
