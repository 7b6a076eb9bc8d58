// Reference-order CONV2D / CONV3D / DEPTHWISE_CONV2D / TRANSPOSE_CONV2D /
// MATMUL / MATMUL_T kernels.
//
// One thread per output element runs the reference's loop nest
// (ConvNd::accumulate, src/ops/conv.rs:149-181; Depthwise::accumulate,
// :234-266; Transpose::accumulate, :337-372; Dims::run,
// src/ops/matmul.rs:80-95) with its accumulator
// semantics (src/ops/accum.rs): int32 wrap, INT48 clamp, sequential fp32
// without contraction, and the FP16/BF16 accumulators that round the product
// and/or the sum. Float results are therefore bit-identical to the
// reference. These kernels serve every type combination the MFMA kernels do
// not (int16 inputs, FP32/FP8 operands, FP16/BF16 accumulators, F16-output
// MATMUL) and the opt-in bit-exact float mode.
#include "kcommon.h"

#pragma clang fp contract(off)

namespace tosa {
namespace kern {
namespace {

__device__ __forceinline__ float fmac(int kind, float acc, float a, float b)
{
    switch (kind) {
    case ACC_F16: {
        const float p = round_fmt(a * b, FMT_F16);
        return round_fmt(acc + p, FMT_F16);
    }
    case ACC_BF16: {
        const float p = round_fmt(a * b, FMT_BF16);
        return round_fmt(acc + p, FMT_BF16);
    }
    case ACC_F16U: return round_fmt(acc + a * b, FMT_F16);
    case ACC_BF16U: return round_fmt(acc + a * b, FMT_BF16);
    default: return acc + a * b;
    }
}

__device__ __forceinline__ int64_t clamp48(int64_t v)
{
    const int64_t lo = -(int64_t(1) << 47), hi = (int64_t(1) << 47) - 1;
    return v < lo ? lo : (v > hi ? hi : v);
}

__global__ void direct_conv_kernel(DirectConvDesc d, const void* x, const void* w, const void* bias, void* out,
                                   int64_t total)
{
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int oc = int(idx % d.oc);
    int64_t r = idx / d.oc;
    const int ox = int(r % d.ow);
    r /= d.ow;
    const int oy = int(r % d.oh);
    r /= d.oh;
    const int oz = int(r % d.od);
    const int b = int(r / d.od);
    const bool is_int = d.acc == ACC_I32 || d.acc == ACC_I64;
    const int nch = d.depthwise ? 1 : d.c;  // channels summed per tap
    const int ci = d.depthwise ? oc / d.m : 0;
    const int mi = d.depthwise ? oc % d.m : 0;
    uint32_t a32 = 0;
    uint64_t a64 = 0;
    float af = 0.0f;
    // Kernel positions row-major (kz, ky, kx), channels innermost (CONV3D:
    // ConvNd::accumulate over three spatial dimensions).
    for (int kz = 0; kz < d.kd; kz++) {
        const int z = oz * d.sz + kz * d.dz - d.pf;
        if (z < 0 || z >= d.id)
            continue;
        for (int ky = 0; ky < d.kh; ky++) {
            const int y = oy * d.sy + ky * d.dy - d.pt;
            if (y < 0 || y >= d.ih)
                continue;
            for (int kx = 0; kx < d.kw; kx++) {
                const int xx = ox * d.sx + kx * d.dx - d.pl;
                if (xx < 0 || xx >= d.iw)
                    continue;
                const int64_t xbase = (((int64_t(b) * d.id + z) * d.ih + y) * d.iw + xx) * d.c;
                for (int c = 0; c < nch; c++) {
                    int64_t xi, wi;
                    if (d.depthwise) {
                        xi = xbase + ci;
                        wi = ((int64_t(ky) * d.kw + kx) * d.c + ci) * d.m + mi;
                    } else {
                        xi = xbase + c;
                        wi = (((int64_t(oc) * d.kd + kz) * d.kh + ky) * d.kw + kx) * d.c + c;
                    }
                    if (is_int) {
                        const int64_t xv = load_int(x, xi, d.xe) - d.zp_x;
                        const int64_t wv = load_int(w, wi, d.we) - d.zp_w;
                        if (d.acc == ACC_I32)
                            a32 += uint32_t(int32_t(xv)) * uint32_t(int32_t(wv));
                        else
                            a64 += uint64_t(xv) * uint64_t(wv);
                    } else {
                        const float xv = load_float(x, xi, d.xe) - d.fzp_x;
                        const float wv = load_float(w, wi, d.we) - d.fzp_w;
                        af = fmac(d.acc, af, xv, wv);
                    }
                }
            }
        }
    }
    const int64_t bi = d.bias_len == 1 ? 0 : oc;
    if (is_int) {
        const int64_t bv = load_int(bias, bi, d.be);
        if (d.acc == ACC_I32)
            static_cast<int32_t*>(out)[idx] = int32_t(a32 + uint32_t(int32_t(bv)));
        else
            static_cast<int64_t*>(out)[idx] = clamp48(int64_t(a64 + uint64_t(bv)));
    } else {
        const float bv = load_float(bias, bi, d.be);
        const float o = round_fmt(round_fmt(af, d.out_fmt) + bv, d.out_fmt);
        store_float(out, idx, d.out_fmt, o);
    }
}

// TRANSPOSE_CONV2D in the reference's gather form (Transpose::accumulate,
// src/ops/conv.rs:337-372): output (oy, ox) reads input
// ((oy - out_pad_top - ky) / sy, (ox - out_pad_left - kx) / sx) where the
// division is exact and the position in range; ky, kx, then channels.
__global__ void direct_tconv_kernel(DirectConvDesc d, const void* x, const void* w, const void* bias, void* out,
                                    int64_t total)
{
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int oc = int(idx % d.oc);
    int64_t r = idx / d.oc;
    const int ox = int(r % d.ow);
    r /= d.ow;
    const int oy = int(r % d.oh);
    const int b = int(r / d.oh);
    const bool is_int = d.acc == ACC_I32 || d.acc == ACC_I64;
    const int iy = oy - d.pt, ix = ox - d.pl;
    uint32_t a32 = 0;
    uint64_t a64 = 0;
    float af = 0.0f;
    for (int ky = 0; ky < d.kh; ky++) {
        const int y = iy - ky;
        if (y < 0 || y >= d.ih * d.sy || y % d.sy != 0)
            continue;
        for (int kx = 0; kx < d.kw; kx++) {
            const int xx = ix - kx;
            if (xx < 0 || xx >= d.iw * d.sx || xx % d.sx != 0)
                continue;
            const int64_t xbase = ((int64_t(b) * d.ih + y / d.sy) * d.iw + xx / d.sx) * d.c;
            const int64_t wbase = ((int64_t(oc) * d.kh + ky) * d.kw + kx) * d.c;
            for (int c = 0; c < d.c; c++) {
                if (is_int) {
                    const int64_t xv = load_int(x, xbase + c, d.xe) - d.zp_x;
                    const int64_t wv = load_int(w, wbase + c, d.we) - d.zp_w;
                    if (d.acc == ACC_I32)
                        a32 += uint32_t(int32_t(xv)) * uint32_t(int32_t(wv));
                    else
                        a64 += uint64_t(xv) * uint64_t(wv);
                } else {
                    const float xv = load_float(x, xbase + c, d.xe) - d.fzp_x;
                    const float wv = load_float(w, wbase + c, d.we) - d.fzp_w;
                    af = fmac(d.acc, af, xv, wv);
                }
            }
        }
    }
    const int64_t bi = d.bias_len == 1 ? 0 : oc;
    if (is_int) {
        const int64_t bv = load_int(bias, bi, d.be);
        if (d.acc == ACC_I32)
            static_cast<int32_t*>(out)[idx] = int32_t(a32 + uint32_t(int32_t(bv)));
        else
            static_cast<int64_t*>(out)[idx] = clamp48(int64_t(a64 + uint64_t(bv)));
    } else {
        const float bv = load_float(bias, bi, d.be);
        const float o = round_fmt(round_fmt(af, d.out_fmt) + bv, d.out_fmt);
        store_float(out, idx, d.out_fmt, o);
    }
}

__global__ void direct_matmul_kernel(DirectMatmulDesc d, const void* a, const void* b, void* out, int64_t total)
{
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int col = int(idx % d.w);
    int64_t r = idx / d.w;
    const int row = int(r % d.h);
    const int n = int(r / d.h);
    const int64_t abase = (int64_t(n) * d.h + row) * d.c;
    // b[., k, col]: at bbase + k * bstep (Dims::b_index, src/ops/matmul.rs:74-77)
    const int64_t nb = d.b_broadcast ? 0 : n;
    const int64_t bbase = d.b_transposed ? (nb * d.w + col) * d.c : nb * d.c * d.w + col;
    const int64_t bstep = d.b_transposed ? 1 : d.w;
    if (d.acc == ACC_I32 || d.acc == ACC_I64) {
        uint32_t a32 = 0;
        uint64_t a64 = 0;
        for (int k = 0; k < d.c; k++) {
            const int64_t av = load_int(a, abase + k, d.ae) - d.zp_a;
            const int64_t bv = load_int(b, bbase + int64_t(k) * bstep, d.be) - d.zp_b;
            if (d.acc == ACC_I32)
                a32 += uint32_t(int32_t(av)) * uint32_t(int32_t(bv));
            else
                a64 += uint64_t(av) * uint64_t(bv);
        }
        if (d.acc == ACC_I32)
            static_cast<int32_t*>(out)[idx] = int32_t(a32);
        else
            static_cast<int64_t*>(out)[idx] = clamp48(int64_t(a64));
    } else {
        float acc = 0.0f;
        for (int k = 0; k < d.c; k++) {
            const float av = round_fmt(load_float(a, abase + k, d.ae), d.out_fmt);
            const float bv = round_fmt(load_float(b, bbase + int64_t(k) * bstep, d.be), d.out_fmt);
            acc = fmac(d.acc, acc, av, bv);
        }
        store_float(out, idx, d.out_fmt, acc);
    }
}

}  // namespace

void direct_conv(const DirectConvDesc& d, const void* x, const void* w, const void* bias, void* out,
                 hipStream_t stream)
{
    const int64_t total = int64_t(d.n) * d.od * d.oh * d.ow * d.oc;
    if (total <= 0)
        return;
    if (d.transpose)
        hipLaunchKernelGGL(direct_tconv_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, stream, d, x, w, bias,
                           out, total);
    else
        hipLaunchKernelGGL(direct_conv_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, stream, d, x, w, bias, out,
                           total);
}

void direct_matmul(const DirectMatmulDesc& d, const void* a, const void* b, void* out, hipStream_t stream)
{
    const int64_t total = int64_t(d.batch) * d.h * d.w;
    if (total > 0)
        hipLaunchKernelGGL(direct_matmul_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, stream, d, a, b, out,
                           total);
}

}  // namespace kern
}  // namespace tosa
