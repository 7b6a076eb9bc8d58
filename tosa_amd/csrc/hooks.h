// Interpreter hooks: the reference's InterpreterHook trait, HookSet and the
// built-in collectors (src/stats.rs:1-298), with two device-path additions a
// hook can declare: needs_sync() (its post_op must see the operator's kernels
// finished, e.g. to time them) and reads_data() (it may read element values,
// so fused-away intermediates must be materialised for it).
#pragma once

#include <chrono>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "tensor.h"

namespace tosa {

struct OpInfo {
    uint32_t op;
    size_t op_index;
};

using TensorRefs = std::vector<const Tensor*>;

class InterpreterHook {
public:
    virtual ~InterpreterHook() = default;
    virtual void pre_op(const OpInfo&, const TensorRefs&) {}
    virtual void post_op(const OpInfo&, const TensorRefs&, const TensorRefs&) {}
    virtual void on_tensor_alloc(const std::string&, const Shape&, DType, size_t) {}
    virtual void on_tensor_free(const std::string&, size_t) {}
    virtual bool needs_sync() const { return false; }
    virtual bool reads_data() const { return false; }
    virtual bool is_noop() const { return false; }
};

class NoopHook : public InterpreterHook {
public:
    bool is_noop() const override { return true; }
};

// src/stats.rs:19-76: dispatches to every hook in insertion order.
class HookSet : public InterpreterHook {
public:
    void add(std::unique_ptr<InterpreterHook> h) { hooks_.push_back(std::move(h)); }
    std::vector<std::unique_ptr<InterpreterHook>>& hooks() { return hooks_; }
    void pre_op(const OpInfo& o, const TensorRefs& in) override;
    void post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out) override;
    void on_tensor_alloc(const std::string& n, const Shape& s, DType t, size_t b) override;
    void on_tensor_free(const std::string& n, size_t b) override;
    bool needs_sync() const override;
    bool reads_data() const override;

private:
    std::vector<std::unique_ptr<InterpreterHook>> hooks_;
};

struct OpStats {
    uint64_t count = 0;
    double total_time = 0;  // seconds
    uint64_t total_input_elements = 0;
    uint64_t total_output_elements = 0;
};

// src/stats.rs:113-195. Times each operator on the host between pre_op and
// post_op; on this path post_op follows a stream synchronisation, so the time
// covers the operator's kernels.
class StatsCollector : public InterpreterHook {
public:
    std::map<std::string, OpStats> op_stats;
    size_t peak_memory_bytes = 0;
    size_t current_memory_bytes = 0;
    uint64_t total_ops_executed = 0;

    std::string summary() const;
    void pre_op(const OpInfo&, const TensorRefs&) override;
    void post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out) override;
    void on_tensor_alloc(const std::string&, const Shape&, DType, size_t bytes) override;
    void on_tensor_free(const std::string&, size_t bytes) override;
    bool needs_sync() const override { return true; }

private:
    bool started_ = false;
    std::chrono::steady_clock::time_point start_;
};

// src/stats.rs:200-263.
class FlopCounter : public InterpreterHook {
public:
    uint64_t total_flops = 0;
    std::map<std::string, uint64_t> flops_by_op;
    void post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out) override;
};

struct TraceEntry {
    std::string op;
    size_t op_index;
    std::vector<Shape> input_shapes, output_shapes;
    double elapsed = 0;  // always zero, as in the reference
};

// src/stats.rs:266-298.
class OpTrace : public InterpreterHook {
public:
    std::vector<TraceEntry> entries;
    void post_op(const OpInfo& o, const TensorRefs& in, const TensorRefs& out) override;
};

}  // namespace tosa
