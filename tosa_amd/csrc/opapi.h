// Op-level entry points (no graph): argument bundle, validated call and
// launch shared by the C ABI functions in capi.cpp.
#pragma once

#include <cstdint>
#include <vector>

#include <hip/hip_runtime.h>

#include "kernels.h"

struct tosa_rescale_i32;

namespace tosa {

// The arguments of tosa_conv2d_i8 (include/tosa_mi355x.h).
struct ConvI8Args {
    const int8_t* x = nullptr;
    const int64_t* x_shape = nullptr;
    const int8_t* w = nullptr;
    const int64_t* w_shape = nullptr;
    const int32_t* bias = nullptr;
    int64_t bias_len = 0;
    int32_t input_zp = 0, weight_zp = 0;
    const int32_t* pad = nullptr;
    const int32_t* stride = nullptr;
    const int32_t* dilation = nullptr;
    const tosa_rescale_i32* rescale = nullptr;
    void* out = nullptr;
    uint32_t* device_error = nullptr;
    void* stream = nullptr;
};

// A validated call: the kernel descriptor, the RESCALE (host fields; its
// device multiplier/shift live in the workspace) and the workspace layout.
struct ConvI8Call {
    kern::ConvI8Desc d;
    kern::RescaleDev rs;
    bool has_rs = false;
    bool epi_ok = true;              // the fused epilogue takes the RESCALE
    std::vector<int32_t> params;     // multipliers, then shifts, as int32
    int64_t out_shape[4] = {0, 0, 0, 0};
    int64_t count = 0;               // output elements
    int64_t params_off = 0, tab_off = 0, wpack_off = 0, tmp_off = 0;
    int64_t wpack_bytes = 0;
    int64_t workspace = 0;           // bytes of device workspace the call needs
};

// Checks the arguments (throws Error with the reference's kinds) and plans
// the call.
ConvI8Call prepare_conv2d_i8(const ConvI8Args& a);
// Enqueues the table, weight-pack and convolution kernels (and the RESCALE
// when the epilogue cannot take it) on `s`, with `ws` holding c.workspace
// bytes whose multiplier/shift words are already in place.
void launch_conv2d_i8(const ConvI8Call& c, uint8_t* ws, void* out, uint32_t* err, hipStream_t s);
// tosa_conv2d_i8: workspace from the stream's pool.
void conv2d_i8(const ConvI8Args& a, int64_t* out_shape);
// tosa_conv2d_i8_noalloc: workspace in the per-GPU static scratch array.
void conv2d_i8_noalloc(const ConvI8Args& a, int64_t* out_shape);

// The arguments of tosa_matmul_i8 (include/tosa_mi355x.h).
struct MatmulI8OpArgs {
    const int8_t* a = nullptr;
    const int64_t* a_shape = nullptr;  // {N, H, C}
    const int8_t* b = nullptr;
    const int64_t* b_shape = nullptr;  // {N, C, W}
    int32_t a_zp = 0, b_zp = 0;
    const tosa_rescale_i32* rescale = nullptr;
    void* out = nullptr;
    uint32_t* device_error = nullptr;
    void* stream = nullptr;
};
// tosa_matmul_i8: workspace (RESCALE words, epilogue table) from the
// stream's pool.
void matmul_i8(const MatmulI8OpArgs& a, int64_t* out_shape);

}  // namespace tosa
