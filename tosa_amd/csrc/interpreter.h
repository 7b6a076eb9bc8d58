// The public C++ API, mirroring the reference's src/lib.rs and
// src/interpreter.rs: Interpreter::{new, from_flatbuffer, graph, run} and the
// run_graph* convenience functions.
#pragma once

#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "exec.h"
#include "hooks.h"
#include "ir.h"

namespace tosa {

using TensorMap = std::unordered_map<std::string, TensorPtr>;

// Highest tensor rank supported (src/interpreter.rs:150-152).
constexpr size_t MAX_RANK = 6;

// What every run of one block shares, built once per graph: the tensor
// definitions by name, a dense id per operand/result name, and each
// operator's distinct input ids and output ids.
struct BlockIndex {
    ExecState::DefMap defs, const_defs;
    std::string rank_error;  // non-empty: the block holds a tensor above MAX_RANK
    std::unordered_map<std::string, int> ids;
    std::vector<std::vector<int>> op_inputs;   // distinct, per operator (empty for CONST)
    std::vector<std::vector<int>> op_outputs;  // in operand order, per operator
    static BlockIndex build(const BasicBlock& b);
};

// The ready queue's starting state for one set of input names: which ids are
// available, how many distinct inputs each operator still misses, the
// operators waiting on each id (graph order) and the initial queue.
struct Schedule {
    std::unordered_set<std::string> input_names;
    std::vector<char> available;
    std::vector<size_t> missing;
    std::vector<std::vector<size_t>> waiting;
    std::vector<size_t> queue;
};

class Interpreter {
public:
    explicit Interpreter(Graph graph);                              // src/interpreter.rs:109
    static Interpreter from_flatbuffer(const uint8_t* data, size_t len);  // :113
    const Graph& graph() const { return graph_; }                   // :118

    // src/interpreter.rs:122-147. Inputs are shared, not consumed; the
    // returned tensors are device-resident.
    TensorMap run(const TensorMap& inputs, InterpreterHook& hook) const;
    TensorMap run(const TensorMap& inputs, InterpreterHook& hook, const RunOptions& opts) const;

private:
    std::shared_ptr<const Schedule> schedule_for(const TensorMap& inputs) const;

    struct ScheduleCache {
        std::mutex mu;
        std::shared_ptr<const Schedule> last;
    };

    Graph graph_;
    mutable std::unique_ptr<ConstCache> consts_;
    FusionPlan plan_;
    BlockIndex index_;
    mutable std::unique_ptr<ScheduleCache> sched_;
};

// Process-wide defaults for RunOptions (set through the C ABI or the
// TOSA_MI355X_FUSION / TOSA_MI355X_STRICT_FLOAT environment variables).
RunOptions& default_run_options();

TensorMap run_graph(const uint8_t* data, size_t len, const TensorMap& inputs);                       // src/lib.rs:20
TensorMap run_graph_with_stats(const uint8_t* data, size_t len, const TensorMap& inputs, StatsCollector& stats);  // :26
TensorMap run_graph_with_hooks(const uint8_t* data, size_t len, const TensorMap& inputs, InterpreterHook& hooks);  // :36

}  // namespace tosa
