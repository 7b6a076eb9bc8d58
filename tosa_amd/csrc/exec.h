// Execution state of one Interpreter::run (the reference's InterpreterState,
// src/interpreter.rs:9-102) plus what the device path adds: a per-graph cache
// of decoded, device-resident constants, the stream, and the bookkeeping of
// fused operator chains.
#pragma once

#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "device.h"
#include "ir.h"
#include "kernels.h"
#include "tensor.h"

namespace tosa {

struct RunOptions {
    bool fusion = true;         // fold RESCALE/CLAMP/residual chains into one kernel
    bool strict_float = false;  // float CONV2D/MATMUL in the reference's sequential order
    // Pipelined runs: run() returns once its kernels are enqueued, without
    // synchronising or reading the error word; REQUIRE failures of any
    // deferred run are reported by the next synchronize().
    bool deferred = false;
};

// CONST payloads decoded once per graph. Their storages become
// device-resident on first use and stay so for later runs: weights cross
// PCIe once per Interpreter, not once per run.
class ConstCache {
public:
    StoragePtr get(const TensorDef& def);

private:
    std::mutex mu_;
    std::unordered_map<const TensorDef*, StoragePtr> map_;
};

// Static fusion opportunities of a block, found once per graph.
struct FusionPlan {
    // head op -> RESCALE op consuming its int32 output (or -1)
    std::vector<int> rescale_after;
    // RESCALE op -> CLAMP op consuming its output (or -1)
    std::vector<int> clamp_after;
    // ADD op whose two operands are RESCALEs of int8 tensors and whose result
    // feeds one RESCALE -> that RESCALE (or -1)
    std::vector<int> residual_tail;
    // RESCALE op whose output feeds such an ADD only
    std::vector<bool> residual_input;
    // Convolution whose fused RESCALE (no CLAMP) feeds only such a residual
    // RESCALE: its launch may wait for the ADD and carry the residual in its
    // epilogue
    std::vector<bool> residual_head;

    static FusionPlan build(const BasicBlock& b);
};

class ExecState {
public:
    const BasicBlock* block = nullptr;
    using DefMap = std::unordered_map<std::string, const TensorDef*>;
    std::unordered_map<std::string, TensorPtr> tensors;
    // Built once per graph by the Interpreter and shared by its runs.
    const DefMap* defs = nullptr;
    const DefMap* const_defs = nullptr;  // outputs of CONST ops
    ConstCache* consts = nullptr;
    const FusionPlan* plan = nullptr;
    RunOptions opts;
    // Outputs already produced by a fused kernel, keyed by tensor name; the
    // owning operator picks them up when the scheduler reaches it.
    std::unordered_map<std::string, TensorPtr> pending;

    TensorPtr get(const std::string& name) const;  // Error(ERR_TENSOR_NOT_FOUND)
    void set(const TensorPtr& t) { tensors[t->name] = t; }
    const TensorDef* find_def(const std::string& name) const;
    bool is_const(const std::string& name) const { return const_defs->count(name) != 0; }
    // An operand of a consumer that has not run yet: a present tensor or a
    // CONST output (decoded from the graph); null otherwise.
    TensorPtr resolve(const std::string& name) const;
    // The thread's stream, acquired (and its error word cleared) on the
    // first kernel launch of the run: graphs that fail validation or hold
    // only constants never touch the device.
    Stream& stream() const
    {
        if (!stream_) {
            stream_ = &thread_stream();
            if (!opts.deferred)
                clear_error_word(*stream_);
        }
        return *stream_;
    }
    bool has_stream() const { return stream_ != nullptr; }
    uint32_t* err() const { return stream().err; }
    hipStream_t s() const { return stream().s; }

private:
    mutable Stream* stream_ = nullptr;
};

// Evaluate one operator (src/ops/mod.rs:22-150).
void dispatch(ExecState& st, const Operator& op, size_t index);

}  // namespace tosa
