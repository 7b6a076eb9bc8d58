// Core types of the MI355X TOSA execution path: element types, operator
// codes, errors.
//
// Element types and operator codes use the numeric values of the TOSA
// FlatBuffer schema (schema/tosa.fbs:26-46 and :88-191), which is also what
// the C ABI exchanges. The reference keeps its own Rust enums
// (src/ir.rs:5-27, :120-242) mapped from those codes; the names returned by
// op_name() are the reference's Op::name() strings (src/ir.rs:352-457).
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace tosa {

enum DType : uint32_t {
    DT_UNKNOWN = 0,
    DT_BOOL = 1,
    DT_INT4 = 2,
    DT_INT8 = 3,
    DT_INT16 = 4,
    DT_INT32 = 5,
    DT_INT48 = 6,
    DT_FP32 = 7,
    DT_FP16 = 8,
    DT_BF16 = 9,
    DT_SHAPE = 10,
    DT_FP8E4M3 = 11,
    DT_FP8E5M2 = 12,
    DT_FP6E2M3 = 13,
    DT_FP6E3M2 = 14,
    DT_FP4E2M1 = 15,
    DT_FP8UE8M0 = 16,
    DT_INT64 = 17,
    DT_MXINT8 = 18,
    DT_FP64 = 64,  // host-only; never produced from a graph
};

// Map a schema code to a DType; unknown codes become DT_UNKNOWN
// (src/ir.rs:29-51).
DType dtype_from_code(uint32_t code);
const char* dtype_name(DType t);

// Bytes per element as held in memory: INT4 unpacked one per byte, INT48
// and SHAPE as int64 (src/ir.rs:53-64).
size_t dtype_size(DType t);
bool dtype_is_int(DType t);    // src/ir.rs:70-72
bool dtype_is_float(DType t);  // src/ir.rs:66-68

// Operator codes (schema/tosa.fbs:88-191).
enum OpCode : uint32_t {
    OP_UNKNOWN = 0,
    OP_ARGMAX = 1,
    OP_AVG_POOL2D = 2,
    OP_CONV2D = 3,
    OP_CONV3D = 4,
    OP_DEPTHWISE_CONV2D = 5,
    OP_FFT2D = 6,
    OP_MATMUL = 7,
    OP_MAX_POOL2D = 8,
    OP_RFFT2D = 9,
    OP_TRANSPOSE_CONV2D = 10,
    OP_CLAMP = 11,
    OP_ADD = 15,
    OP_SUB = 30,
    OP_MUL = 28,
    OP_CONCAT = 55,
    OP_PAD = 56,
    OP_RESHAPE = 57,
    OP_TRANSPOSE = 61,
    OP_CAST = 65,
    OP_RESCALE = 66,
    OP_CONST = 67,
    OP_IDENTITY = 68,
    OP_CUSTOM = 69,
    OP_COND_IF = 70,
    OP_WHILE_LOOP = 71,
    OP_VARIABLE = 72,
    OP_VARIABLE_WRITE = 73,
    OP_VARIABLE_READ = 74,
    OP_CONST_SHAPE = 75,
    OP_MATMUL_T = 100,
    OP_ARGMIN = 101,
    OP_LAST = 101,
};

// The reference's Op::name(); "UNKNOWN" for codes outside the schema.
const char* op_name(uint32_t op);

// Error kinds: the reference's Error enum (src/error.rs:4-31) plus Device,
// for failures of the GPU runtime itself.
enum ErrorKind : int {
    ERR_OK = 0,
    ERR_DESERIALIZE = 1,
    ERR_UNSUPPORTED_OP = 2,
    ERR_TENSOR_NOT_FOUND = 3,
    ERR_DTYPE_MISMATCH = 4,
    ERR_SHAPE_MISMATCH = 5,
    ERR_BROADCAST = 6,
    ERR_GRAPH = 7,
    ERR_CONTROL_FLOW = 8,
    ERR_IO = 9,
    ERR_DEVICE = 10,
};

struct Error : std::runtime_error {
    ErrorKind kind;
    Error(ErrorKind k, const std::string& m) : std::runtime_error(m), kind(k) {}
};

// ERROR_IF violation of an operator (src/ops/common.rs:9-11).
inline Error invalid(const std::string& op, const std::string& msg) { return Error(ERR_GRAPH, op + ": " + msg); }

using Shape = std::vector<int64_t>;
std::string shape_str(const Shape& s);
int64_t shape_count(const Shape& s);  // product; 1 for rank 0

}  // namespace tosa
