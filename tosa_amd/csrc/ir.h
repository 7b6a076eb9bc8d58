// Graph IR: what a `.tosa` FlatBuffer holds, as the reference parses it
// (src/ir.rs:461-589). Attributes are decoded by union type, exactly as
// Graph::parse_attribute does (src/ir.rs:673-885): an operator whose union
// holds another operator's table gets that table's attribute, and the
// operator's own evaluation then rejects it as "missing attribute".
#pragma once

#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "core.h"

namespace tosa {

enum class AttrKind {
    None,
    CondIf,
    WhileLoop,
    Conv2d,
    Conv3d,
    DepthwiseConv2d,
    TransposeConv2d,
    Pool2d,
    ArgMax,
    Reduce,
    Dim,
    Fft2d,
    AssertEqualShape,
    NanPropagation,
    Concat,
    Transpose,
    Clamp,
    ArithmeticRightShift,
    Rescale,
    Reverse,
    Resize,
};

// NanPropagationMode (schema/tosa.fbs:53-57) as the reference holds it.
enum NanMode : uint32_t { NAN_UNKNOWN = 0, NAN_PROPAGATE = 1, NAN_IGNORE = 2 };
// RoundingMode (schema/tosa.fbs:59-64).
enum RoundingMode : uint32_t { ROUND_UNKNOWN = 0, ROUND_SINGLE = 1, ROUND_INEXACT = 2, ROUND_DOUBLE = 3 };

struct OpAttribute {
    AttrKind kind = AttrKind::None;
    std::vector<int32_t> pad, stride, dilation, kernel, out_pad, perms;
    DType acc_type = DT_UNKNOWN;
    NanMode nan_mode = NAN_PROPAGATE;
    std::vector<uint8_t> min_val, max_val;  // CLAMP bounds, serialized in the input type
    bool scale32 = false, per_channel = false, input_unsigned = false, output_unsigned = false;
    RoundingMode rounding_mode = ROUND_UNKNOWN;
    int32_t axis = 0;
    bool flag = false;  // inverse (FFT2D), round (ARS), allow_broadcast
    std::string graph_a, graph_b;
};

struct TensorDef {
    std::string name;
    std::vector<int32_t> shape;
    DType dtype = DT_UNKNOWN;
    bool has_data = false;
    std::vector<uint8_t> data;
    bool is_variable = false;
};

struct Operator {
    uint32_t op = OP_UNKNOWN;
    std::vector<std::string> inputs, outputs;
    OpAttribute attr;
};

struct BasicBlock {
    std::string name;
    std::vector<Operator> operators;
    std::vector<TensorDef> tensors;
    std::vector<std::string> inputs, outputs;
};

struct Region {
    std::string name;
    std::vector<BasicBlock> blocks;
};

struct Graph {
    std::vector<Region> regions;

    // src/ir.rs:587-614; throws Error(ERR_DESERIALIZE) on malformed input.
    static Graph from_flatbuffer(const uint8_t* data, size_t len);
    const BasicBlock* main_block() const;                 // src/ir.rs:887-889
    const BasicBlock* find_block(const std::string&) const;  // src/ir.rs:891-908
};

}  // namespace tosa
