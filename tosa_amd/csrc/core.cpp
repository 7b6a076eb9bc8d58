#include "core.h"

namespace tosa {

DType dtype_from_code(uint32_t code)
{
    if (code <= DT_MXINT8)
        return static_cast<DType>(code);
    return DT_UNKNOWN;
}

const char* dtype_name(DType t)
{
    switch (t) {
    case DT_BOOL: return "BOOL";
    case DT_INT4: return "INT4";
    case DT_INT8: return "INT8";
    case DT_INT16: return "INT16";
    case DT_INT32: return "INT32";
    case DT_INT48: return "INT48";
    case DT_FP32: return "FP32";
    case DT_FP16: return "FP16";
    case DT_BF16: return "BF16";
    case DT_SHAPE: return "SHAPE";
    case DT_FP8E4M3: return "FP8E4M3";
    case DT_FP8E5M2: return "FP8E5M2";
    case DT_FP6E2M3: return "FP6E2M3";
    case DT_FP6E3M2: return "FP6E3M2";
    case DT_FP4E2M1: return "FP4E2M1";
    case DT_FP8UE8M0: return "FP8UE8M0";
    case DT_INT64: return "INT64";
    case DT_MXINT8: return "MXINT8";
    case DT_FP64: return "FP64";
    default: return "UNKNOWN";
    }
}

size_t dtype_size(DType t)
{
    switch (t) {
    case DT_BOOL:
    case DT_INT4:
    case DT_INT8:
    case DT_FP8E4M3:
    case DT_FP8E5M2:
    case DT_FP6E2M3:
    case DT_FP6E3M2:
    case DT_FP4E2M1:
    case DT_FP8UE8M0:
    case DT_MXINT8: return 1;
    case DT_INT16:
    case DT_FP16:
    case DT_BF16: return 2;
    case DT_INT32:
    case DT_FP32: return 4;
    case DT_INT48:
    case DT_INT64:
    case DT_FP64:
    case DT_SHAPE: return 8;
    default: return 0;
    }
}

bool dtype_is_int(DType t)
{
    return t == DT_INT4 || t == DT_INT8 || t == DT_INT16 || t == DT_INT32 || t == DT_INT48 || t == DT_INT64;
}

bool dtype_is_float(DType t)
{
    return t == DT_FP8E4M3 || t == DT_FP8E5M2 || t == DT_FP16 || t == DT_BF16 || t == DT_FP32 || t == DT_FP64;
}

static const char* const kOpNames[] = {
    "UNKNOWN", "ARGMAX", "AVG_POOL2D", "CONV2D", "CONV3D", "DEPTHWISE_CONV2D", "FFT2D", "MATMUL", "MAX_POOL2D",
    "RFFT2D", "TRANSPOSE_CONV2D", "CLAMP", "ERF", "SIGMOID", "TANH", "ADD", "ARITHMETIC_RIGHT_SHIFT", "BITWISE_AND",
    "BITWISE_OR", "BITWISE_XOR", "INTDIV", "LOGICAL_AND", "LOGICAL_LEFT_SHIFT", "LOGICAL_RIGHT_SHIFT", "LOGICAL_OR",
    "LOGICAL_XOR", "MAXIMUM", "MINIMUM", "MUL", "POW", "SUB", "TABLE", "ABS", "BITWISE_NOT", "CEIL", "CLZ", "COS",
    "EXP", "FLOOR", "LOG", "LOGICAL_NOT", "NEGATE", "RECIPROCAL", "RSQRT", "SIN", "SELECT", "EQUAL", "GREATER",
    "GREATER_EQUAL", "REDUCE_ALL", "REDUCE_ANY", "REDUCE_MAX", "REDUCE_MIN", "REDUCE_PRODUCT", "REDUCE_SUM",
    "CONCAT", "PAD", "RESHAPE", "REVERSE", "SLICE", "TILE", "TRANSPOSE", "GATHER", "SCATTER", "RESIZE", "CAST",
    "RESCALE", "CONST", "IDENTITY", "CUSTOM", "COND_IF", "WHILE_LOOP", "VARIABLE", "VARIABLE_WRITE",
    "VARIABLE_READ", "CONST_SHAPE", "MATMUL_T_BLOCK_SCALED", "CAST_FROM_BLOCK_SCALED", "CAST_TO_BLOCK_SCALED",
    "DIM", "CONCAT_SHAPE", "ADD_SHAPE", "SUB_SHAPE", "MUL_SHAPE", "SLICE_SHAPE", "EXP2_SHAPE", "LOG2_CEIL_SHAPE",
    "LOG2_FLOOR_SHAPE", "MAX_SHAPE", "MIN_SHAPE", "MOD_SHAPE", "DIV_CEIL_SHAPE", "DIV_FLOOR_SHAPE",
    "ASSERT_EQUAL_SHAPE", "CONV2D_BLOCK_SCALED", "MAX_POOL2D_ADAPTIVE", "AVG_POOL2D_ADAPTIVE",
    "RESHAPE_BLOCK_SCALED", "ROW_GATHER_BLOCK_SCALED", "ROW_GATHER", "MATMUL_T", "ARGMIN",
};

const char* op_name(uint32_t op)
{
    if (op <= OP_LAST)
        return kOpNames[op];
    return "UNKNOWN";
}

std::string shape_str(const Shape& s)
{
    std::string r = "[";
    for (size_t i = 0; i < s.size(); i++) {
        if (i)
            r += ", ";
        r += std::to_string(s[i]);
    }
    return r + "]";
}

int64_t shape_count(const Shape& s)
{
    int64_t n = 1;
    for (int64_t d : s)
        n *= d;
    return n;
}

}  // namespace tosa
