// The public C++ API, mirroring the reference's src/lib.rs and
// src/interpreter.rs: Interpreter::{new, from_flatbuffer, graph, run} and the
// run_graph* convenience functions.
#pragma once

#include <memory>
#include <string>
#include <unordered_map>

#include "exec.h"
#include "hooks.h"
#include "ir.h"

namespace tosa {

using TensorMap = std::unordered_map<std::string, TensorPtr>;

// Highest tensor rank supported (src/interpreter.rs:150-152).
constexpr size_t MAX_RANK = 6;

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
    Graph graph_;
    mutable std::unique_ptr<ConstCache> consts_;
    FusionPlan plan_;
};

// Process-wide defaults for RunOptions (set through the C ABI or the
// TOSA_MI355X_FUSION / TOSA_MI355X_STRICT_FLOAT environment variables).
RunOptions& default_run_options();

TensorMap run_graph(const uint8_t* data, size_t len, const TensorMap& inputs);                       // src/lib.rs:20
TensorMap run_graph_with_stats(const uint8_t* data, size_t len, const TensorMap& inputs, StatsCollector& stats);  // :26
TensorMap run_graph_with_hooks(const uint8_t* data, size_t len, const TensorMap& inputs, InterpreterHook& hooks);  // :36

}  // namespace tosa
