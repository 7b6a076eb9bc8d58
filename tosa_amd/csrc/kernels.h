// Host-side launchers of the gfx950 kernels. Every pointer is a device
// pointer; every launcher enqueues on `stream` and returns immediately.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace tosa {
namespace kern {

// n / d for 0 <= n < 2^31 with a multiply-high and a shift (d >= 1).
struct FastDiv {
    uint32_t d = 1, m = 1, s = 0;
    FastDiv() = default;
    explicit FastDiv(uint32_t div);
};

// RESCALE applied per element (src/ops/type_conv.rs:171-188), optionally
// followed by a CLAMP (src/ops/elementwise.rs:328-334). Multiplier and shift
// are validated on the host before launch (multiplier >= 0, shift in
// [2, 62] unless INEXACT), so kernels only check the value-dependent
// REQUIRE conditions.
struct RescaleDev {
    const int32_t* mult = nullptr;  // [channels]
    const int32_t* shift = nullptr; // [channels]
    int32_t channels = 1;           // per-channel: channel = flat index % channels
    int32_t per_channel = 0;
    int32_t scale32 = 1;            // 0: 16-bit multiplier (apply_scale_16)
    int32_t rounding = 1;           // 1 SINGLE, 2 INEXACT, 3 DOUBLE
    int32_t in_bits = 32;           // input type width, for unsigned extension
    int32_t in_unsigned = 0;
    int64_t in_zp = 0, out_zp = 0;  // already extended
    int64_t lo = 0, hi = 0;         // output range (signed or unsigned)
    int32_t has_clamp = 0;
    int64_t clamp_lo = 0, clamp_hi = 0;
    int32_t out_bytes = 1;          // 1, 2 or 4
    int32_t max_shift = 62;         // largest shift over the channels (host-checked)
    int32_t min_shift = 2;          // smallest shift over the channels
};

// Epilogue of a GEMM-shaped operator.
enum Epilogue : int32_t {
    EPI_I32 = 0,      // int32 accumulator + bias, written as int32
    EPI_RESCALE = 1,  // int32 accumulator + bias, then RescaleDev
    EPI_FLOAT = 2,    // fp32 accumulator: out = round(round(acc) + bias)
};

// Float storage formats used by the float epilogues.
enum FloatFmt : int32_t { FMT_F32 = 0, FMT_F16 = 1, FMT_BF16 = 2, FMT_FP8E4M3 = 3, FMT_FP8E5M2 = 4 };

enum GemmElem : int32_t { ELEM_I8 = 0, ELEM_BF16 = 1, ELEM_F16 = 2 };

// Implicit-GEMM convolution or batched matmul on MFMA.
//   conv:   x NHWC [n,ih,iw,ic], w OHWI [oc,kh,kw,ic] -> out NHWC [n,oh,ow,oc]
//   matmul: a [n,h,c], b [n,c,w] -> out [n,h,w]
struct GemmDesc {
    int32_t is_conv = 1;
    GemmElem elem = ELEM_I8;
    // conv geometry
    int32_t n = 1, ih = 1, iw = 1, ic = 1, oc = 1, kh = 1, kw = 1, oh = 1, ow = 1;
    int32_t pt = 0, pl = 0, sy = 1, sx = 1, dy = 1, dx = 1;
    // matmul geometry
    int32_t batch = 1, h = 1, c = 1, w = 1;
    // int8 zero points: x/a side and w/b side
    int32_t zp_x = 0, zp_w = 0;
    const int32_t* wsum = nullptr;  // conv: per-oc sum of weights (needed when zp_x != 0)
    const void* bias = nullptr;     // conv only: int32 (int path) or f32 values (float path)
    int32_t bias_len = 0;
    Epilogue epi = EPI_I32;
    RescaleDev rs;
    FloatFmt out_fmt = FMT_F32;
};

void gemm(const GemmDesc& d, const void* x, const void* w, void* out, uint32_t* err, hipStream_t stream);

// Per-output-channel sum of an OHWI int8 weight: wsum[o] = sum_k w[o][k]
// (mod 2^32).
void weight_sums_i8(const int8_t* w, int32_t oc, int32_t k, int32_t* wsum, hipStream_t stream);

// ---------------------------------------------------------------------------
// int8 CONV2D on MFMA with a table-driven epilogue (conv_i8.hip)
// ---------------------------------------------------------------------------
struct ConvI8Desc {
    const int8_t* x = nullptr;     // NHWC [n, ih, iw, ic]
    const int8_t* w = nullptr;     // OHWI [oc, kh, kw, ic]
    const int32_t* bias = nullptr; // [bias_len], bias_len 1 or oc
    int32_t bias_len = 1;
    int32_t n = 1, ih = 1, iw = 1, ic = 1, oc = 1, kh = 1, kw = 1, oh = 1, ow = 1;
    int32_t pt = 0, pl = 0, sy = 1, sx = 1, dy = 1, dx = 1;
    int32_t zp_x = 0, zp_w = 0;
    // DEPTHWISE_CONV2D with depth multiplier 1: w is [kh, kw, ic, 1] and
    // oc == ic.
    int32_t depthwise = 0;
    // Weights packed by conv_i8_wpack (when conv_i8_wpack_bytes > 0); the
    // stride-1 halo kernel runs only with them.
    const int8_t* wpack = nullptr;
    // Independent pointwise problems (1x1 stride-1 unpadded CONV2D only):
    // x [batch][n oh ow][ic], w [batch][oc][ic], out [batch][n oh ow][oc] and
    // the table [batch][conv_i8_table_stride(oc)]. A batched MATMUL runs as
    // this with B transposed to rows of C bytes.
    int32_t batch = 1;
    // The epilogue table proved that no value can fail apply_scale_32's
    // range REQUIRE (conv_i8_table_range_safe), so the kernels skip it.
    bool range_safe = false;
    // Quantised residual folded into the epilogue (conv_i8_residual_ok):
    // the int8 result y of the fused RESCALE goes on through
    // RESCALE(y) + RESCALE(skip) -> ADD -> RESCALE, and only that is stored.
    const int8_t* res_skip = nullptr;  // [pixels][oc] int8, the other ADD operand's source
    const void* res_tab = nullptr;     // conv_i8_residual_table output
    int32_t res_za = 0, res_zb = 0;    // input zero points of RESCALE(y) and RESCALE(skip)
    int32_t res_clo = 0, res_chi = 0;  // final output range (the last RESCALE's, narrowed to its CLAMP)
};
// Geometry and alignment the kernels handle: CONV2D 1x1 stride-1 unpadded
// with ic % 16 == 0, any other CONV2D geometry with ic % 64 == 0;
// DEPTHWISE_CONV2D with ic % 16 == 0 and at most 12 taps; 16-byte aligned
// x (and w for CONV2D).
bool conv_i8_fast_supported(const ConvI8Desc& d);
// RESCALEs the fused epilogue handles: scale32 with SINGLE or DOUBLE
// rounding, signed input with zero point 0 (the only legal one for int32),
// and an output zero point the table can fold into its rounding constants
// (|zp| 2^max_shift <= 2^60).
bool conv_i8_fast_epilogue_ok(const RescaleDev& rs);
// Whether a 1x1 stride-1 int8 CONV2D whose fused RESCALE `rs` gives int8
// (no CLAMP) can carry the quantised residual RESCALE(y; ra) +
// RESCALE(skip; rb) -> ADD -> RESCALE(ro) in its epilogue: ra and rb int8
// -> int32 with shifts >= 9 (so their REQUIREs cannot fail), ro int32 ->
// int8 with SINGLE/DOUBLE rounding and a foldable output zero point, a
// multiple of 4 and at most 1024 channels, a 4-byte aligned skip tensor.
bool conv_i8_residual_ok(const ConvI8Desc& d, const RescaleDev& rs, const RescaleDev& ra, const RescaleDev& rb,
                         const RescaleDev& ro, const void* skip);
// Per-channel constants of the three residual RESCALEs, built on the device
// (CONV_I8_RES_WORDS int32 per channel).
constexpr int CONV_I8_RES_WORDS = 20;
void conv_i8_residual_table(const RescaleDev& ra, const RescaleDev& rb, const RescaleDev& ro, int32_t channels,
                            void* out, hipStream_t stream);
// Per-channel epilogue table (8 int32 per output channel, then 4 int32 of
// the input zero point's byte, then one int32 per channel) built on the
// device from w, bias, the zero points and, when `rs` is given, the RESCALE
// multiplier and shift.
constexpr int CONV_I8_TABLE_WORDS = 8;
inline int64_t conv_i8_table_words(int32_t oc) { return int64_t(CONV_I8_TABLE_WORDS + 1) * oc + 4; }
// int32 words between the tables of consecutive batches (64-byte aligned).
inline int64_t conv_i8_table_stride(int32_t oc) { return (conv_i8_table_words(oc) + 15) / 16 * 16; }
// Words of a table for all of d's batches.
inline int64_t conv_i8_table_words(int32_t oc, int32_t batch)
{
    return int64_t(batch - 1) * conv_i8_table_stride(oc) + conv_i8_table_words(oc);
}
void conv_i8_table(const ConvI8Desc& d, const RescaleDev* rs, void* tab, hipStream_t stream);
// True when the table (complete on the device) marks every channel whose
// shift is below 32 as unable to fail apply_scale_32's range REQUIRE: the
// channel's bound |bias| + max|x - zx| sum_k |w - zw| lies below 2^(shift-1).
// Copies the table to the host (synchronous).
bool conv_i8_table_range_safe(const ConvI8Desc& d, const void* tab);
// Bytes of the packed weight layout of the stride-1 halo kernel for `d`, 0
// when that kernel does not run for `d`; conv_i8_wpack writes it from d.w.
int64_t conv_i8_wpack_bytes(const ConvI8Desc& d);
// Output channels per block of that layout (0 when it does not apply).
int conv_i8_wpack_block(const ConvI8Desc& d);
void conv_i8_wpack(const ConvI8Desc& d, void* wp, hipStream_t stream);
// Convolutions that conv_i8_fast_supported rejects only for their channel
// alignment or geometry run as a pointwise GEMM over a materialised im2col:
// X~ [n oh ow][Kp] (Kp = K rounded up to 16; padding taps hold the input
// zero point, columns past K hold 0) and the weights as [oc][Kp] rows
// (zero-filled). The table is still built from the original descriptor.
int32_t conv_i8_im2col_kp(const ConvI8Desc& d);
void conv_i8_im2col(const ConvI8Desc& d, int8_t* xcol, hipStream_t stream);
void conv_i8_rowpad(const int8_t* w, int32_t rows, int32_t k, int32_t kp, int8_t* out, hipStream_t stream);
// MATMUL right operand [batch][c][w] -> [batch][w][c] (c % 16 == 0).
void transpose_b_i8(const int8_t* b, int32_t batch, int32_t c, int32_t w, int8_t* out, hipStream_t stream);
// Compute units of the current device.
int cu_count();
// Batched int8 MATMUL a [batch][H][C] x b [batch][C][W] (+ fused RESCALE)
// in one kernel that reads B in its own layout (matmul_i8_kernel,
// conv_i8.hip); `tab` is conv_i8_table's output for a descriptor with w null
// (no weight sums: the kernel adds -zp_a sum_c b itself). Takes C % 128 == 0,
// W % 16 == 0 and 16-byte aligned operands; false otherwise (nothing done).
bool matmul_i8_direct_applies(int32_t C, int32_t W, const void* a, const void* b);
bool matmul_i8_direct(const int8_t* a, const int8_t* b, int32_t batch, int32_t H, int32_t C, int32_t W, int32_t zp_a,
                      int32_t zp_b, const void* tab, const RescaleDev* rs, bool range_safe, void* out, uint32_t* err,
                      hipStream_t stream);
// Whether int8 3x3 convolutions that fit it run on the row-tile kernel
// (mode 1, the default; mode 2: 64-channel workgroups only) rather than the
// halo kernel (mode 0); all are bit-exact.
// Rows of A per workgroup of the int8 MATMUL kernel (64 or 128).
void set_mm_tile_rows(int rows);
int mm_tile_rows();
void set_conv_rows_mode(int mode);
int conv_rows_mode();
bool conv_rows_enabled();
// 1x1 stride-1 int8 CONV2D with the fused RESCALE to int8 on the streaming
// pointwise kernel, for the shapes it takes (conv_i8.hip: K <= 64 a multiple
// of 8, many pixels); false otherwise.
bool conv_i8_pointwise_stream(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                              hipStream_t stream);
// int8 CONV2D of 3x3 taps over 3 input channels (stride 1 or 2, padding up
// to 2, iw % 4 == 0, oc % 32 == 0) with the fused RESCALE to int8, its im2col
// built in LDS (conv_i8.hip); wpad holds the weights as [oc][32] rows (the 27
// taps, then zeros). False when the shape or epilogue does not fit.
bool conv_i8_stem(const ConvI8Desc& d, const void* tab, const int8_t* wpad, const RescaleDev* rs, void* out,
                  uint32_t* err, hipStream_t stream);
// DEPTHWISE_CONV2D (multiplier 1, ic % 16 == 0, at most 12 taps) over
// LDS-staged input tiles (dw_i8.hip); false when the shape does not fit its
// LDS budget. Same table and epilogue contract as conv_i8_fast.
bool depthwise_i8_lds(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                      hipStream_t stream);
// The same over a persistent grid that loads each (image, rows, channel
// chunk) tile into LDS by direct global -> LDS loads while the previous tile
// computes (dw_i8.hip); false for shapes it does not take (16-byte aligned
// input and weights, tiles within its LDS budget).
bool depthwise_i8_pipe(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                       hipStream_t stream);
// The convolution; `rs` selects the fused RESCALE (+CLAMP) epilogue with the
// table built for the same `rs`, else the int32 output (conv + bias).
void conv_i8_fast(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                  hipStream_t stream);

// ---------------------------------------------------------------------------
// bf16 / fp16 GEMM with fp32 accumulation (gemm_f16.hip)
// ---------------------------------------------------------------------------
// C[b][m][n] = sum_k A[b][m][k] B[b][k][n] (b_kn: B as [K][N], the MATMUL
// right operand) or sum_k A[b][m][k] B[b][n][k] (OHWI 1x1 weights), then
// out = round(round(C) + bias[n]) in out_fmt when a bias is given (the
// CONV2D float epilogue), else C rounded to out_fmt.
struct GemmF16Desc {
    int32_t batch = 1, m = 1, n = 1, k = 1;
    GemmElem elem = ELEM_BF16;
    bool b_kn = true;
    const void* bias = nullptr;  // f32 [bias_len], bias_len 1 or n
    int32_t bias_len = 1;
    FloatFmt out_fmt = FMT_F32;
};
// K a multiple of 64, 16-byte aligned operands, N % 8 == 0 for a [K][N] B,
// every matrix below 2^31 elements.
bool gemm_f16_supported(int64_t batch, int64_t m, int64_t n, int64_t k, bool b_kn, const void* a, const void* b);
void gemm_f16(const GemmF16Desc& d, const void* a, const void* b, void* out, hipStream_t stream);

// bf16 / fp16 CONV2D with fp32 accumulation on the stride-1 halo kernel
// (the int8 headline kernel's float variant): NHWC x, OHWI w, f32 bias,
// out = round(round(acc) + bias) in out_fmt (src/ops/conv.rs:475-496 with
// AccF32). Applies to stride-1 convolutions with ic % 16 == 0, output rows
// of at most 512 pixels and 16-byte aligned x and w:
// conv_f16_halo_wpack_bytes(d) > 0 then, and conv_f16_halo runs with the
// weights that conv_f16_halo_wpack packed into d.wpack.
struct ConvF16Desc {
    const void* x = nullptr;  // bf16 / fp16 [n, ih, iw, ic]
    const void* w = nullptr;  // bf16 / fp16 [oc, kh, kw, ic]
    GemmElem elem = ELEM_BF16;
    int32_t n = 1, ih = 1, iw = 1, ic = 1, oc = 1, kh = 1, kw = 1, oh = 1, ow = 1;
    int32_t pt = 0, pl = 0, sy = 1, sx = 1, dy = 1, dx = 1;
    const float* bias = nullptr;  // [bias_len], bias_len 1 or oc
    int32_t bias_len = 1;
    FloatFmt out_fmt = FMT_F32;
    const void* wpack = nullptr;
};
int64_t conv_f16_halo_wpack_bytes(const ConvF16Desc& d);
// Output channels per block of that packing (0 when the kernel does not apply).
int conv_f16_halo_block(const ConvF16Desc& d);
void conv_f16_halo_wpack(const ConvF16Desc& d, void* wp, hipStream_t stream);
void conv_f16_halo(const ConvF16Desc& d, void* out, hipStream_t stream);

// ---------------------------------------------------------------------------
// Reference-order kernels (one thread per output, the reference's loop
// order and rounding, so float results are bit-identical to a sequential
// evaluation). They cover every type combination the MFMA path does not.
// ---------------------------------------------------------------------------
enum AccKind : int32_t {
    ACC_I32 = 0, ACC_I64 = 1,                 // integer: wrap mod 2^32 / INT48 clamp
    ACC_F32 = 2, ACC_F16 = 3, ACC_BF16 = 4,   // accum.rs AccF32 / AccF16 / AccBf16
    ACC_F16U = 5, ACC_BF16U = 6,              // accum.rs Acc*UnroundedProduct (MATMUL)
};

// Element codes for the direct kernels' operands.
enum ElemCode : int32_t {
    E_I8 = 0, E_I16 = 1, E_I32 = 2, E_I64 = 3,
    E_F32 = 4, E_F16 = 5, E_BF16 = 6, E_FP8E4M3 = 7, E_FP8E5M2 = 8, E_U8 = 9,
};

struct DirectConvDesc {
    int32_t depthwise = 0;
    int32_t n, ih, iw, c, m, oc, kh, kw, oh, ow, pt, pl, sy, sx, dy, dx;  // c = input channels, m = multiplier
    // CONV3D: the depth dimension (input id, kernel kd, output od, front pad
    // pf, stride sz, dilation dz); 1/0 for the 2-D convolutions.
    int32_t id = 1, kd = 1, od = 1, pf = 0, sz = 1, dz = 1;
    // TRANSPOSE_CONV2D (gather form): pt/pl are out_pad top/left (possibly
    // negative), sy/sx the strides; dy/dx unused.
    int32_t transpose = 0;
    ElemCode xe, we, be, oe;  // input, weight, bias and output element codes
    AccKind acc;
    int64_t zp_x = 0, zp_w = 0;   // integer zero points
    float fzp_x = 0, fzp_w = 0;   // float zero points (subtracted as in the reference)
    int32_t bias_len = 1;
    int32_t out_fmt = FMT_F32;    // float output rounding format
};
void direct_conv(const DirectConvDesc& d, const void* x, const void* w, const void* bias, void* out,
                 hipStream_t stream);

struct DirectMatmulDesc {
    int32_t batch, h, c, w;
    int32_t b_transposed = 0;  // MATMUL_T: b is [D][w][c] rather than [batch][c][w]
    int32_t b_broadcast = 0;   // MATMUL_T with D = 1: every batch reads b's only slice
    ElemCode ae, be, oe;
    AccKind acc;
    int64_t zp_a = 0, zp_b = 0;
    int32_t out_fmt = FMT_F32;  // operands are rounded to this format first (matmul.rs:160-162)
};
void direct_matmul(const DirectMatmulDesc& d, const void* a, const void* b, void* out, hipStream_t stream);

// ---------------------------------------------------------------------------
// Bandwidth-bound kernels
// ---------------------------------------------------------------------------

// int8 DEPTHWISE_CONV2D with depth multiplier 1, int32 accumulation and an
// I32 / RESCALE epilogue.
struct DepthwiseDesc {
    int32_t n, ih, iw, c, kh, kw, oh, ow, pt, pl, sy, sx, dy, dx;
    int32_t zp_x = 0, zp_w = 0;
    const int32_t* bias = nullptr;
    int32_t bias_len = 1;
    Epilogue epi = EPI_I32;
    RescaleDev rs;
};
// Shapes the int8 depthwise kernel handles: 1x1, 1x3, 3x1, 2x2 and 3x3 taps,
// channels a multiple of 4. The caller checks this before launching.
bool depthwise_i8_supported(int kh, int kw, int c);
void depthwise_i8(const DepthwiseDesc& d, const int8_t* x, const int8_t* w, void* out, uint32_t* err,
                  hipStream_t stream);

struct PoolDesc {
    int32_t n, ih, iw, c, kh, kw, oh, ow, pt, pl, sy, sx;
    ElemCode xe;
    int64_t in_zp = 0, out_zp = 0, lo = 0, hi = 0;  // integer path
    int32_t acc_fmt = FMT_F32;                       // float path: accumulator rounding
    int32_t out_fmt = FMT_F32;                       // float path: output encoding
};
void avg_pool2d(const PoolDesc& d, const void* x, void* out, uint32_t* err, hipStream_t stream);
// MAX_POOL2D (xe int8/int16 or a float code; out in the same type): `ignore`
// selects NaN mode IGNORE, `lowest` is the float type's lowest value.
void max_pool2d(const PoolDesc& d, bool ignore, float lowest, const void* x, void* out, hipStream_t stream);

// CAST between the element types (src/ops/type_conv.rs:45-80): from/to
// element codes, `from_float` / `to_float` tell integer (BOOL: E_U8) from
// float codes, `to_bool` marks a BOOL result, to_fmt the float output
// format; float -> int saturates at hi/lo when the value reaches hi_bound /
// lo_bound (the bounds rounded to the input's precision).
struct CastDesc {
    ElemCode from, to;
    int32_t from_float = 0, to_float = 0, to_bool = 0;
    int32_t to_fmt = FMT_F32;
    int64_t lo = 0, hi = 0;
    float lo_bound = 0, hi_bound = 0;
};
void cast(const CastDesc& d, const void* x, int64_t count, void* out, hipStream_t stream);

// int16 x as int8 halves: x = 256 hi + (lo + 128), hi = x >> 8.
void split_i16(const int16_t* x, int64_t count, int8_t* hi, int8_t* lo, hipStream_t stream);
// out[i] = clamp48(sum_k coef[k] parts[k][i] + bias), int64 arithmetic;
// bias (INT48 as int64) per channel i % channels, or one value, or null.
void combine_i48(const int32_t* const* parts, const int64_t* coef, int nparts, const int64_t* bias, int32_t bias_len,
                 int32_t channels, int64_t count, int64_t* out, hipStream_t stream);
// combine_i48 followed by the RESCALE `rs` of its result (rs.in_bits 48),
// written in the RESCALE's output type.
void combine_i48_rescale(const int32_t* const* parts, const int64_t* coef, int nparts, const int64_t* bias,
                         int32_t bias_len, int32_t channels, int64_t count, const RescaleDev& rs, void* out,
                         uint32_t* err, hipStream_t stream);

// Standalone RESCALE over `count` elements of element code `xe`.
void rescale(const RescaleDev& rs, ElemCode xe, const void* x, int64_t count, void* out, uint32_t* err,
             hipStream_t stream);

// CLAMP: ints compare as int64; floats use nan_max/nan_min
// (src/ops/common.rs:155-177) and round to the type.
void clamp(ElemCode e, const void* x, int64_t count, int64_t ilo, int64_t ihi, float flo, float fhi, int nan_ignore,
           void* out, hipStream_t stream);

// Broadcasting ADD of rank <= 6 operands (src/ops/elementwise.rs:395-397).
struct BroadcastDesc {
    int32_t rank = 0;
    int64_t out_dims[6] = {1, 1, 1, 1, 1, 1};
    int64_t a_strides[6] = {0}, b_strides[6] = {0};  // element strides, 0 on broadcast dims
};
void add(ElemCode e, const BroadcastDesc& bd, const void* a, const void* b, void* out, int64_t count,
         hipStream_t stream);

// Residual block of a quantised graph, fused: out = RESCALE_o(RESCALE_a(a) +
// RESCALE_b(b)) where RESCALE_a/b take int8 to int32 and RESCALE_o takes
// int32 to int8 (equal shapes, no broadcast).
void residual_add_i8(const RescaleDev& ra, const RescaleDev& rb, const RescaleDev& ro, const int8_t* a,
                     const int8_t* b, int64_t count, int64_t channels, void* out, uint32_t* err,
                     hipStream_t stream);

// TRANSPOSE of a rank <= 6 tensor with elements of `esize` bytes.
void transpose(const void* x, void* out, int32_t esize, int32_t rank, const int64_t* out_dims,
               const int64_t* in_strides_permuted, int64_t count, hipStream_t stream);

}  // namespace kern
}  // namespace tosa
