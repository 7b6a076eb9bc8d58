// int8 CONV2D as an implicit GEMM on CDNA4 MFMA (v_mfma_i32_16x16x64_i8),
// with the per-channel epilogue (bias, zero-point corrections, RESCALE,
// CLAMP) driven by a precomputed table.
//
// Replaces ConvNd::accumulate::<AccI32> (src/ops/conv.rs:149-181), the bias
// add (src/ops/conv.rs:464) and, when fused, eval_rescale
// (src/ops/type_conv.rs:174-188) with apply_scale_32 (src/ops/quant.rs:17-32)
// and eval_clamp (src/ops/elementwise.rs:328-334).
//
// GEMM view: D[c][p] = sum_k W[c][k] * X~[p][k] over k = (ky*KW + kx)*IC + ic
// (the OHWI weight row order), p = output pixel (n*OH*OW), c = output
// channel. X~ is the im2col view of the NHWC input with padding taps set to
// the input zero point, so that (x~ - zx) vanishes there; the zero points are
// folded into the int32 accumulator (mod 2^32):
//   sum_k (x~ - zx)(w - zw) = sum x~ w - zw sum_k x~ - zx sum_k w + K zx zw.
// The per-channel terms (bias + K zx zw - zx sum_k w) come from the table,
// the per-pixel term zw sum_k x~ from the staged input bytes.
//
// Layout: 256 threads (4 waves) per workgroup compute a BC-channel x
// BP-pixel tile. K advances KC bytes per stage through two LDS buffers whose
// rows hold KC bytes with the 16-byte chunks XOR-swizzled by row, so the
// fragment reads of a wave and the staging writes are free of bank
// conflicts. With IC a multiple of KC every stage lies inside one kernel tap,
// so the tap position (ky, kx, ic0) is uniform across the workgroup and the
// im2col address of a pixel row is its precomputed origin plus a scalar
// offset. The channel rows of the A fragments are interleaved so that each
// lane ends up holding 4*TM consecutive output channels of one pixel, which
// the epilogue stores as one vector.
#include "kcommon.h"

namespace tosa {
namespace kern {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));

struct ConvI8Args {
    const int8_t* x;
    const int8_t* w;
    uint8_t* out;
    const v4i* tab;  // 2 entries per output channel (see conv_i8_table_kernel)
    int32_t M, N, K, IC;
    int32_t ih, iw, kw, ohow, ow, pt, pl, sy, sx, dy, dx;
    FastDiv div_ohow, div_ow;
    int32_t zp_x, zp_w;
    int32_t out_zp;          // RESCALE output zero point
    int32_t zp_lo, zp_hi;    // r + out_zp stays in int32 iff zp_lo <= r <= zp_hi
    int32_t lo, hi;    // output type range
    int32_t clo, chi;  // CLAMP bounds (the output range when there is no CLAMP)
    uint32_t* err;
};

// A 16-byte global load returned by value (a conditional between a load and
// a register value then stays a select of values, not of addresses).
__device__ __forceinline__ v4u ld16(const int8_t* p) { return *reinterpret_cast<const v4u*>(p); }

// Physical 16-byte chunk of logical chunk c in LDS row `row`.
template <int KC>
__device__ __forceinline__ int swz(int row)
{
    if constexpr (KC == 128)
        return (row ^ (row >> 2)) & 7;
    else
        return ((row >> 1) ^ (row >> 3)) & 3;
}

// BC x BP tile, WC x WP waves, KC bytes of K per stage. PW: 1x1 stride-1
// unpadded convolution (a plain GEMM over the NHWC rows; K may be any
// multiple of 16). OB: output bytes (1, 2, 4). RS: RESCALE epilogue (else
// int32 + bias). ZW: weight zero point is nonzero.
template <int BC, int BP, int WC, int WP, int KC, bool PW, int OB, bool RS, bool ZW>
__global__ void __launch_bounds__(256, 2) conv_i8_kernel(ConvI8Args A)
{
    constexpr int TM = BC / WC / 16;
    constexpr int TN = BP / WP / 16;
    constexpr int CPR = KC / 16;              // 16-byte chunks per LDS row
    constexpr int RPP = 256 / CPR;            // rows staged per pass of the workgroup
    constexpr int PCH = BP / RPP;             // pixel rows per thread
    constexpr int QCH = (BC + RPP - 1) / RPP; // weight rows per thread
    static_assert(WC * WP == 4 && TM >= 1 && TN >= 1 && BP % RPP == 0, "tile shape");

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* const sA = smem;                 // [2][BC][KC]
    uint8_t* const sB = smem + 2 * BC * KC;   // [2][BP][KC]
    int32_t* const s_rowsum = reinterpret_cast<int32_t*>(smem);  // after the main loop

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_c0 = (wave / WP) * (BC / WC);
    const int wave_p0 = (wave % WP) * (BP / WP);
    const int m0 = blockIdx.x * BP;
    const int n0 = blockIdx.y * BC;
    const int ch = tid % CPR;
    const int r0 = tid / CPR;

    // ---- im2col origin of the pixel rows this thread stages ---------------
    int32_t pbase[PCH], piy[PCH], pix[PCH];
#pragma unroll
    for (int p = 0; p < PCH; p++) {
        const int m = m0 + r0 + RPP * p;
        if constexpr (PW) {
            pbase[p] = m < A.M ? m * A.IC : -1;
            piy[p] = pix[p] = 0;
        } else {
            const int mm = m < A.M ? m : 0;
            const int b = fdiv(mm, A.div_ohow);
            const int rem = mm - b * A.ohow;
            const int oy = fdiv(rem, A.div_ow);
            const int ox = rem - oy * A.ow;
            pbase[p] = b * A.ih * A.iw * A.IC;
            piy[p] = m < A.M ? oy * A.sy - A.pt : -(1 << 29);  // rows past M read padding
            pix[p] = ox * A.sx - A.pl;
        }
    }
    // Weight rows past N re-read row N-1: their products land in output
    // channels that are never stored.
    int32_t wbase[QCH];
#pragma unroll
    for (int q = 0; q < QCH; q++) {
        const int oc = n0 + r0 + RPP * q;
        wbase[q] = (oc < A.N ? oc : A.N - 1) * A.K;
    }

    const uint32_t zf = uint32_t(uint8_t(A.zp_x)) * 0x01010101u;
    const v4u zfill = v4u{zf, zf, zf, zf};
    const v4u zero = v4u{0, 0, 0, 0};
    int32_t rsum[PCH];
#pragma unroll
    for (int p = 0; p < PCH; p++)
        rsum[p] = 0;

    v4u pr[PCH], qr[QCH];
    // Stage `kk` (K offset); (ky, kx, ic0): its kernel tap and channel offset.
    auto load = [&](int kk, int ky, int kx, int ic0) {
        const int kc = kk + ch * 16;
#pragma unroll
        for (int p = 0; p < PCH; p++) {
            // Every lane loads (from offset 0 when its tap is outside the
            // input or the row is past M) and then selects the value.
            if constexpr (PW) {
                const bool ok = pbase[p] >= 0 && kc < A.K;
                const v4u v = ld16(A.x + (ok ? pbase[p] + kc : 0));
                pr[p] = ok ? v : zero;
            } else {
                const int iy = piy[p] + ky * A.dy;
                const int ix = pix[p] + kx * A.dx;
                const bool ok = unsigned(iy) < unsigned(A.ih) && unsigned(ix) < unsigned(A.iw);
                const v4u v = ld16(A.x + (ok ? pbase[p] + (iy * A.iw + ix) * A.IC + ic0 + ch * 16 : 0));
                pr[p] = ok ? v : zfill;
            }
            if constexpr (ZW) {
                int32_t s = rsum[p];
                s = __builtin_amdgcn_sdot4(int(pr[p].x), 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4(int(pr[p].y), 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4(int(pr[p].z), 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4(int(pr[p].w), 0x01010101, s, false);
                rsum[p] = s;
            }
        }
        // Chunks past K (pointwise K not a multiple of KC) re-read the row's
        // last 16 bytes; the pixel side is zero there, so they add nothing.
        const int kw_off = kc < A.K ? kc : A.K - 16;
#pragma unroll
        for (int q = 0; q < QCH; q++)
            qr[q] = ld16(A.w + wbase[q] + kw_off);
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PCH; p++) {
            const int row = r0 + RPP * p;
            *reinterpret_cast<v4u*>(sB + buf * BP * KC + row * KC + ((ch ^ swz<KC>(row)) << 4)) = pr[p];
        }
#pragma unroll
        for (int q = 0; q < QCH; q++) {
            const int row = r0 + RPP * q;
            if (BC % RPP == 0 || row < BC)
                *reinterpret_cast<v4u*>(sA + buf * BC * KC + row * KC + ((ch ^ swz<KC>(row)) << 4)) = qr[q];
        }
    };

    // The tile's epilogue table, staged in LDS behind the stage buffers.
    v4i* const s_tab = reinterpret_cast<v4i*>(smem + 2 * (BC + BP) * KC);
    for (int i = tid; i < 2 * BC; i += 256) {
        const int c = n0 + (i >> 1);
        s_tab[i] = A.tab[2 * (c < A.N ? c : A.N - 1) + (i & 1)];
    }

    v4i acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
            acc[a][b] = v4i{0, 0, 0, 0};

    const int nst = (A.K + KC - 1) / KC;
    // Tap of the next stage to load (uniform).
    int ky = 0, kx = 0, ic0 = 0;
    auto advance = [&]() {
        if constexpr (!PW) {
            ic0 += KC;
            if (ic0 == A.IC) {
                ic0 = 0;
                if (++kx == A.kw) {
                    kx = 0;
                    ky++;
                }
            }
        }
    };
    load(0, ky, kx, ic0);
    advance();
    store(0);
    __syncthreads();

    const int j16 = lane & 15;
    const int grp = lane >> 4;
    for (int s = 0; s < nst; s++) {
        const int buf = s & 1;
        if (s + 1 < nst) {
            load((s + 1) * KC, ky, kx, ic0);
            advance();
        }
        const uint8_t* a = sA + buf * BC * KC;
        const uint8_t* b = sB + buf * BP * KC;
#pragma unroll
        for (int ks = 0; ks < KC / 64; ks++) {
            const int c = ks * 4 + grp;
            v4i af[TM], bf[TN];
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                const int row = wave_c0 + (j16 >> 2) * (4 * TM) + 4 * tm + (j16 & 3);
                af[tm] = *reinterpret_cast<const v4i*>(a + row * KC + ((c ^ swz<KC>(row)) << 4));
            }
#pragma unroll
            for (int tn = 0; tn < TN; tn++) {
                const int row = wave_p0 + 16 * tn + j16;
                bf[tn] = *reinterpret_cast<const v4i*>(b + row * KC + ((c ^ swz<KC>(row)) << 4));
            }
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
                    acc[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[tm], bf[tn], acc[tm][tn], 0, 0, 0);
        }
        if (s + 1 < nst)
            store(buf ^ 1);
        __syncthreads();
    }

    // ---- per-pixel weight-zero-point term ---------------------------------
    if constexpr (ZW) {
#pragma unroll
        for (int p = 0; p < PCH; p++) {
            int32_t v = rsum[p];
#pragma unroll
            for (int o = 1; o < CPR; o <<= 1)
                v += __shfl_xor(v, o);
            if (ch == 0)
                s_rowsum[r0 + RPP * p] = v;
        }
        __syncthreads();
    }

    // ---- epilogue ----------------------------------------------------------
    const int cl0 = wave_c0 + grp * 4 * TM;  // first tile channel held by this lane
    const int c0 = n0 + cl0;
    bool bad_range = false, bad_zp = false;
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
        // One channel group at a time: keeps the scheduler from hoisting every
        // group's table reads (32 registers each) to the top.
        __builtin_amdgcn_sched_barrier(0);
        v4i t0[4], t1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            t0[i] = s_tab[2 * (cl0 + 4 * tm + i)];
            if constexpr (RS)
                t1[i] = s_tab[2 * (cl0 + 4 * tm + i) + 1];
        }
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            // Four outputs at a time (bounds the 64-bit temporaries in flight).
            __builtin_amdgcn_sched_barrier(0);
            int32_t zwx = 0;
            if constexpr (ZW)
                zwx = int32_t(uint32_t(A.zp_w) * uint32_t(s_rowsum[wave_p0 + 16 * tn + j16]));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int32_t x = int32_t(uint32_t(acc[tm][tn][i]) + uint32_t(t0[i].x) - uint32_t(zwx));
                if constexpr (RS) {
                    // apply_scale_32: the value must lie in [-2^(s-1), 2^(s-1)),
                    // a condition on int32 values only for shifts below 32
                    // (t0.z = min(s - 1, 31)).
                    const int32_t hi_bits = x >> t0[i].z;
                    bad_range |= uint32_t(hi_bits + 1) > 1u;
                    const int64_t rnd = x >= 0 ? ((int64_t(t1[i].y) << 32) | uint32_t(t1[i].x))
                                               : ((int64_t(t1[i].w) << 32) | uint32_t(t1[i].z));
                    // With the value in range and 0 <= multiplier < 2^31 the
                    // scaled result always fits int32 (|r| <= 2^30 + 1), so
                    // apply_scale_32's result REQUIRE cannot fail here.
                    const int64_t r = (int64_t(x) * int64_t(t0[i].y) + rnd) >> t0[i].w;
                    const int32_t r32 = int32_t(r);
                    bad_zp |= (r32 < A.zp_lo) | (r32 > A.zp_hi);
                    int32_t v = r32 + A.out_zp;
                    v = v < A.lo ? A.lo : (v > A.hi ? A.hi : v);
                    v = v < A.clo ? A.clo : (v > A.chi ? A.chi : v);
                    // Materialise the 32-bit result here: otherwise the
                    // 64-bit intermediates are sunk towards the final stores
                    // and held in registers across every group.
                    asm volatile("" : "+v"(v));
                    acc[tm][tn][i] = v;
                } else {
                    acc[tm][tn][i] = x;
                }
            }
        }
    }

#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int m = m0 + wave_p0 + 16 * tn + j16;
        if (m >= A.M)
            continue;
        const int64_t o = int64_t(m) * A.N + c0;
        uint8_t* dst = A.out + o * OB;
        constexpr int VB = 4 * TM * OB;  // bytes this lane holds for the pixel
        if (c0 + 4 * TM <= A.N && ((o * OB) % (VB < 16 ? VB : 16)) == 0) {
            if constexpr (OB == 1) {
                uint32_t wd[TM];
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
                    wd[tm] = (uint32_t(acc[tm][tn][0]) & 0xFF) | ((uint32_t(acc[tm][tn][1]) & 0xFF) << 8) |
                             ((uint32_t(acc[tm][tn][2]) & 0xFF) << 16) | (uint32_t(acc[tm][tn][3]) << 24);
                if constexpr (TM == 4)
                    *reinterpret_cast<v4u*>(dst) = v4u{wd[0], wd[1], wd[2], wd[3]};
                else if constexpr (TM == 2)
                    *reinterpret_cast<v2u*>(dst) = v2u{wd[0], wd[1]};
                else
                    *reinterpret_cast<uint32_t*>(dst) = wd[0];
            } else if constexpr (OB == 2) {
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
                    *reinterpret_cast<v2u*>(dst + 8 * tm) =
                        v2u{(uint32_t(acc[tm][tn][0]) & 0xFFFF) | (uint32_t(acc[tm][tn][1]) << 16),
                            (uint32_t(acc[tm][tn][2]) & 0xFFFF) | (uint32_t(acc[tm][tn][3]) << 16)};
            } else {
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
                    *reinterpret_cast<v4i*>(dst + 16 * tm) = acc[tm][tn];
            }
        } else {
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (c0 + 4 * tm + i >= A.N)
                        continue;
                    const int e = 4 * tm + i;
                    if constexpr (OB == 1)
                        dst[e] = uint8_t(acc[tm][tn][i]);
                    else if constexpr (OB == 2)
                        reinterpret_cast<uint16_t*>(dst)[e] = uint16_t(acc[tm][tn][i]);
                    else
                        reinterpret_cast<int32_t*>(dst)[e] = acc[tm][tn][i];
                }
        }
    }
    if (bad_range)
        atomicOr(A.err, DERR_SCALE_RANGE);
    if (bad_zp)
        atomicOr(A.err, DERR_RESCALE_I32);
}

// One wave per output channel:
//   tab[2c]   = {bias + K zx zw - zx sum_k w[c][k] (mod 2^32), multiplier,
//                min(shift - 1, 31), shift}
//   tab[2c+1] = {rounding constant for values >= 0 (int64, lo/hi),
//                rounding constant for values < 0 (int64, lo/hi)}
// The rounding constants are apply_scale_32's 2^(s-1), plus or minus 2^30
// under double rounding for shifts above 31 (src/ops/quant.rs:26-29).
__global__ void conv_i8_table_kernel(const int8_t* w, int32_t N, int32_t K, const int32_t* bias, int32_t bias_len,
                                     int32_t zx, int32_t zw, const int32_t* mult, const int32_t* shift,
                                     int32_t per_channel, int32_t dbl, v4i* tab)
{
    const int c = blockIdx.x;
    const int lane = threadIdx.x;
    int32_t s = 0;
    if (zx != 0)
        for (int k = lane; k < K; k += 64)
            s += w[int64_t(c) * K + k];
    for (int off = 32; off > 0; off >>= 1)
        s += __shfl_xor(s, off);
    if (lane != 0)
        return;
    uint32_t add = bias ? uint32_t(bias[bias_len == 1 ? 0 : c]) : 0u;
    add += uint32_t(K) * uint32_t(zx) * uint32_t(zw);
    add -= uint32_t(zx) * uint32_t(s);
    int32_t m = 0, sh = 2;
    if (mult) {
        m = mult[per_channel ? c : 0];
        sh = shift[per_channel ? c : 0];
    }
    const int64_t half = int64_t(1) << (sh - 1);
    const int64_t d = (dbl && sh > 31) ? (int64_t(1) << 30) : 0;
    const int64_t rp = half + d, rn = half - d;
    tab[2 * c] = v4i{int32_t(add), m, sh - 1 < 31 ? sh - 1 : 31, sh};
    tab[2 * c + 1] = v4i{int32_t(uint32_t(uint64_t(rp))), int32_t(uint64_t(rp) >> 32),
                         int32_t(uint32_t(uint64_t(rn))), int32_t(uint64_t(rn) >> 32)};
}

template <int BC, int BP, int WC, int WP, int KC, bool PW, int OB, bool RS, bool ZW>
void launch(const ConvI8Args& a, hipStream_t s)
{
    auto kfn = conv_i8_kernel<BC, BP, WC, WP, KC, PW, OB, RS, ZW>;
    constexpr size_t lds = size_t(2) * (BC + BP) * KC + size_t(32) * BC;
    static_assert(lds >= 4 * BP, "rowsum scratch");
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      int(lds)),
                  "conv_i8 LDS size");
        return true;
    }();
    (void)attr;
    dim3 grid((a.M + BP - 1) / BP, (a.N + BC - 1) / BC);
    hipLaunchKernelGGL(kfn, grid, dim3(256), lds, s, a);
}

template <int BC, int BP, int WC, int WP, int KC, bool PW>
void launch_epi(const ConvI8Args& a, int ob, bool rs, bool zw, hipStream_t s)
{
    if (!rs) {
        if (zw)
            launch<BC, BP, WC, WP, KC, PW, 4, false, true>(a, s);
        else
            launch<BC, BP, WC, WP, KC, PW, 4, false, false>(a, s);
        return;
    }
#define TOSA_CONV_OB(OBV)                                          \
    if (zw)                                                        \
        launch<BC, BP, WC, WP, KC, PW, OBV, true, true>(a, s);     \
    else                                                           \
        launch<BC, BP, WC, WP, KC, PW, OBV, true, false>(a, s);
    if (ob == 1) {
        TOSA_CONV_OB(1)
    } else if (ob == 2) {
        TOSA_CONV_OB(2)
    } else {
        TOSA_CONV_OB(4)
    }
#undef TOSA_CONV_OB
}

template <int KC, bool PW>
void launch_tile(const ConvI8Args& a, int ob, bool rs, bool zw, hipStream_t s)
{
    if (a.N > 64)
        launch_epi<128, 128, 2, 2, KC, PW>(a, ob, rs, zw, s);
    else if (a.N > 32)
        launch_epi<64, 256, 1, 4, KC, PW>(a, ob, rs, zw, s);
    else if (a.N > 16)
        launch_epi<32, 256, 1, 4, KC, PW>(a, ob, rs, zw, s);
    else
        launch_epi<16, 256, 1, 4, KC, PW>(a, ob, rs, zw, s);
}

}  // namespace

bool conv_i8_fast_supported(const ConvI8Desc& d)
{
    const bool pw = d.kh == 1 && d.kw == 1 && d.sy == 1 && d.sx == 1 && d.pt == 0 && d.pl == 0 && d.ih == d.oh &&
                    d.iw == d.ow;
    const bool aligned = (reinterpret_cast<uintptr_t>(d.x) % 16 == 0) && (reinterpret_cast<uintptr_t>(d.w) % 16 == 0);
    if (!aligned)
        return false;
    if (pw)
        return d.ic % 16 == 0;
    return d.ic % 64 == 0;
}

void conv_i8_table(const ConvI8Desc& d, const RescaleDev* rs, void* tab, hipStream_t stream)
{
    if (d.oc <= 0)
        return;
    const int32_t K = d.kh * d.kw * d.ic;
    hipLaunchKernelGGL(conv_i8_table_kernel, dim3(d.oc), dim3(64), 0, stream, d.w, d.oc, K, d.bias, d.bias_len,
                       d.zp_x, d.zp_w, rs ? rs->mult : nullptr, rs ? rs->shift : nullptr,
                       rs ? rs->per_channel : 0, rs ? int32_t(rs->rounding == 3) : 0, static_cast<v4i*>(tab));
}

bool conv_i8_fast_epilogue_ok(const RescaleDev& rs)
{
    return rs.scale32 && (rs.rounding == 1 || rs.rounding == 3) && !rs.in_unsigned && rs.in_zp == 0 &&
           (rs.out_bytes == 1 || rs.out_bytes == 2 || rs.out_bytes == 4);
}

void conv_i8_fast(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                  hipStream_t stream)
{
    ConvI8Args a{};
    a.x = d.x;
    a.w = d.w;
    a.out = static_cast<uint8_t*>(out);
    a.tab = static_cast<const v4i*>(tab);
    a.M = d.n * d.oh * d.ow;
    a.N = d.oc;
    a.K = d.kh * d.kw * d.ic;
    a.IC = d.ic;
    a.ih = d.ih;
    a.iw = d.iw;
    a.kw = d.kw;
    a.ohow = d.oh * d.ow;
    a.ow = d.ow;
    a.pt = d.pt;
    a.pl = d.pl;
    a.sy = d.sy;
    a.sx = d.sx;
    a.dy = d.dy;
    a.dx = d.dx;
    a.div_ohow = FastDiv(uint32_t(a.ohow));
    a.div_ow = FastDiv(uint32_t(d.ow));
    a.zp_x = d.zp_x;
    a.zp_w = d.zp_w;
    a.err = err;
    int ob = 4;
    if (rs) {
        a.out_zp = int32_t(rs->out_zp);
        a.zp_lo = rs->out_zp < 0 ? int32_t(INT32_MIN - rs->out_zp) : INT32_MIN;
        a.zp_hi = rs->out_zp > 0 ? int32_t(INT32_MAX - rs->out_zp) : INT32_MAX;
        a.lo = int32_t(rs->lo);
        a.hi = int32_t(rs->hi);
        a.clo = rs->has_clamp ? int32_t(rs->clamp_lo) : a.lo;
        a.chi = rs->has_clamp ? int32_t(rs->clamp_hi) : a.hi;
        ob = rs->out_bytes;
    }
    if (a.M <= 0 || a.N <= 0)
        return;
    const bool zw = d.zp_w != 0;
    const bool pw = d.kh == 1 && d.kw == 1 && d.sy == 1 && d.sx == 1 && d.pt == 0 && d.pl == 0 && d.ih == d.oh &&
                    d.iw == d.ow;
    if (pw) {
        if (a.K >= 128)
            launch_tile<128, true>(a, ob, rs != nullptr, zw, stream);
        else
            launch_tile<64, true>(a, ob, rs != nullptr, zw, stream);
    } else if (d.ic % 128 == 0) {
        launch_tile<128, false>(a, ob, rs != nullptr, zw, stream);
    } else {
        launch_tile<64, false>(a, ob, rs != nullptr, zw, stream);
    }
}

}  // namespace kern
}  // namespace tosa
