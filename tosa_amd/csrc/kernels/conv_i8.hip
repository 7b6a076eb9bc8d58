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
#include <algorithm>
#include <atomic>

#include <stdexcept>
#include <type_traits>
#include <vector>

#include "kcommon.h"

namespace tosa {
namespace kern {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef int v2i __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(1))) void gvoid;
typedef __attribute__((address_space(3))) void lvoid;

// What the epilogue needs besides the accumulators.
struct EpiArgs {
    uint8_t* out;            // NHWC [pixels][N]
    int32_t N;               // output channels
    int32_t zp_w;            // weight zero point (per-pixel correction)
    int32_t clo, chi;        // output type range, narrowed to the CLAMP bounds if fused
    uint32_t* err;
    // Some channel's shift is below 32, so apply_scale_32's value-range
    // REQUIRE can fail and is checked (with every shift >= 32 it cannot).
    int32_t range;
    // The rounding constant does not depend on the value's sign (single
    // rounding, or no shift above 31): the tiled epilogue skips the select.
    int32_t one_round;
    // Quantised residual in the epilogue (kernels instantiated with it): the
    // skip tensor (same layout as the output), the input zero points of its
    // two int8 -> int32 RESCALEs, and the final output range (the last
    // RESCALE's type range, narrowed to a fused CLAMP).
    const int8_t* skip;
    int32_t za, zb, rclo, rchi;
};


struct ConvI8Args {
    const int8_t* x;
    const int8_t* w;
    const v4i* tab;  // 2 entries per output channel (see conv_i8_table_kernel)
    int32_t M, N, K, IC;
    int32_t ih, iw, kw, ohow, ow, pt, pl, sy, sx, dy, dx;
    FastDiv div_ohow, div_ow;
    int32_t zp_x;
    EpiArgs E;
    // Pointwise batches (blockIdx.z): strides of x, w and out in bytes and
    // of the table in 16-byte entries.
    int64_t bsx, bsw, bso;
    int32_t bst, batch;
    const int32_t* rtab;  // residual constants, CONV_I8_RES_WORDS per channel (RES kernels)
};

// Median of three (v_med3_i32): clamp of v to [lo, hi] when lo <= hi.
__device__ __forceinline__ int32_t med3(int32_t v, int32_t lo, int32_t hi)
{
    int32_t r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(lo), "v"(hi));
    return r;
}

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

// Bias, zero-point terms, RESCALE and CLAMP of a wave's accumulators, and
// the stores. Lane (grp, j16) holds, for each pixel tile tn, the 4*TM
// consecutive channels starting at tile channel `cl0` of tile pixel
// wave_p0 + 16 tn + j16; `pixel(p)` maps a tile pixel to its output row
// (NHWC pixel index) or -1 when the pixel does not exist.
// apply_scale_32 of a residual RESCALE with per-channel constants m, s and
// the sign-selected rounding constant (output zero point folded in).
__device__ __forceinline__ int32_t res_apply(int32_t x, int32_t m, int32_t s, int64_t rp, int64_t rn)
{
    return int32_t((int64_t(x) * m + (x >= 0 ? rp : rn)) >> s);
}

// RES: the RESCALE result y (int8) goes on through the quantised residual:
// y' = RESCALE(RESCALE(y - za) + RESCALE(skip - zb)) with the constants of
// s_res (CONV_I8_RES_WORDS per tile channel: m, s, rp, rn of each of the
// three RESCALEs, then the last one's value-range bound), and y' is stored.
// CS: tile channels between consecutive channel groups tm of a lane (4: the
// lane's 4 TM channels are consecutive; 16: groups of 4 consecutive channels
// 16 apart, each stored on its own).
template <int TM, int TN, int OB, bool RS, bool ZW, bool RC, bool RES = false, int CS = 4, typename PixelMap>
__device__ __forceinline__ void epilogue(v4i (&acc)[TM][TN], const v4i* s_tab, const int32_t* s_rowsum, int cl0,
                                         int n0, int wave_p0, int j16, const EpiArgs& E, PixelMap pixel,
                                         const int32_t* s_res = nullptr)
{
    static_assert(!RES || (RS && OB == 1), "the residual follows an int8 RESCALE");
    static_assert(CS == 4 || !RES, "the residual stage takes consecutive channels");
    constexpr int WORDS = TM * OB;  // 32-bit words of output per lane and pixel
    const int c0 = n0 + cl0;
    uint32_t res[TN][WORDS];
    // Skip bytes of this lane's channels (four per word), loaded up front.
    uint32_t skw[RES ? TN : 1][RES ? TM : 1];
    uint32_t res_bad = 0;
    if constexpr (RES) {
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            const int m = pixel(wave_p0 + 16 * tn + j16);
#pragma unroll
            for (int tm = 0; tm < TM; tm++)
                skw[tn][tm] = m >= 0 && c0 + 4 * tm < E.N
                                  ? *reinterpret_cast<const uint32_t*>(E.skip + int64_t(m) * E.N + c0 + 4 * tm)
                                  : 0u;
        }
    }
    // Nonzero when a value fails apply_scale_32's range REQUIRE (one bitwise
    // op per value on the VALU).
    uint32_t bad_bits = 0;
    // Table entries of channel group tm (4 channels), read one group ahead:
    // the next group's LDS reads are in flight while this one computes.
    v4i tq0[2][4], tq1[2][RS ? 4 : 1];
    auto tab_load = [&](int tm, int slot) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            tq0[slot][i] = s_tab[2 * (cl0 + CS * tm + i)];
            if constexpr (RS)
                tq1[slot][i] = s_tab[2 * (cl0 + CS * tm + i) + 1];
        }
    };
    tab_load(0, 0);
    // ONE: E.one_round, as a compile-time flag of each copy of the loop (a
    // branch on the uniform kernel argument picks the copy).
    auto groups = [&](auto onec) {
    constexpr bool ONE = decltype(onec)::value;
#pragma unroll
    for (int tm = 0; tm < TM; tm++) {
        // One channel group at a time: keeps the scheduler from hoisting every
        // group's table reads (32 registers each) to the top.
        __builtin_amdgcn_sched_barrier(0);
        if (tm + 1 < TM)
            tab_load(tm + 1, (tm + 1) & 1);
        const v4i* const t0 = tq0[tm & 1];
        const v4i* const t1 = tq1[tm & 1];
        int32_t hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            hi[i] = ~t0[i].z;
        // The group's residual constants (words 0-18 of each channel).
        int32_t rq[4][RES ? 20 : 1];
        if constexpr (RES) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const v4i* q = reinterpret_cast<const v4i*>(s_res + CONV_I8_RES_WORDS * (cl0 + 4 * tm + i));
#pragma unroll
                for (int k = 0; k < 5; k++) {
                    const v4i v = q[k];
                    rq[i][4 * k] = v.x;
                    rq[i][4 * k + 1] = v.y;
                    rq[i][4 * k + 2] = v.z;
                    rq[i][4 * k + 3] = v.w;
                }
            }
        }
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            // Four outputs at a time (bounds the 64-bit temporaries in flight).
            __builtin_amdgcn_sched_barrier(0);
            uint32_t nzwx = 0;  // -zw sum_k x~ of the pixel
            if constexpr (ZW)
                nzwx = uint32_t(-E.zp_w) * uint32_t(s_rowsum[wave_p0 + 16 * tn + j16]);
            int32_t v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int32_t x = int32_t(uint32_t(acc[tm][tn][i]) + uint32_t(t0[i].x) + nzwx);
                if constexpr (RS) {
                    // apply_scale_32: the value must lie in [-2^(s-1), 2^(s-1)),
                    // a condition on int32 values only for shifts below 32
                    // (t0.z = -2^min(s - 1, 31), ~t0.z = 2^min(s - 1, 31) - 1).
                    if constexpr (RC)
                        bad_bits = __builtin_amdgcn_bitop3_b32(bad_bits, uint32_t(med3(x, t0[i].z, hi[i])),
                                                               uint32_t(x), 0xf6);  // bad | (med3 ^ x)
                    const int64_t rp = __builtin_bit_cast(int64_t, v2i{t1[i].x, t1[i].y});
                    const int64_t rn = __builtin_bit_cast(int64_t, v2i{t1[i].z, t1[i].w});
                    // With the value in range and 0 <= multiplier < 2^31 the
                    // scaled result always fits int32 (|r| <= 2^30 + 1), so
                    // apply_scale_32's result REQUIRE cannot fail; rp and rn
                    // carry the output zero point (|zp| <= 2^16), so r is
                    // already RESCALE's r + zp, which fits int32 as well.
                    const int64_t rc = ONE ? rp : (x >= 0 ? rp : rn);
                    const int32_t r = int32_t((int64_t(x) * int64_t(t0[i].y) + rc) >> t0[i].w);
                    // Output range and CLAMP in one step: the CLAMP bounds lie
                    // inside the output type's range, so clamping to the
                    // type and then to [clo, chi] is clamping to [clo, chi].
                    v[i] = med3(r, E.clo, E.chi);
                } else {
                    v[i] = x;
                }
            }
            if constexpr (RES) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int32_t* q = rq[i];
                    const int64_t rpa = __builtin_bit_cast(int64_t, v2i{q[2], q[3]});
                    const int64_t rna = __builtin_bit_cast(int64_t, v2i{q[4], q[5]});
                    const int64_t rpb = __builtin_bit_cast(int64_t, v2i{q[8], q[9]});
                    const int64_t rnb = __builtin_bit_cast(int64_t, v2i{q[10], q[11]});
                    const int64_t rpo = __builtin_bit_cast(int64_t, v2i{q[14], q[15]});
                    const int64_t rno = __builtin_bit_cast(int64_t, v2i{q[16], q[17]});
                    const int32_t va = res_apply(v[i] - E.za, q[0], q[1], rpa, rna);
                    const int32_t sb = int32_t(int8_t(skw[tn][tm] >> (8 * i)));
                    const int32_t vb = res_apply(sb - E.zb, q[6], q[7], rpb, rnb);
                    const int32_t sum = int32_t(uint32_t(va) + uint32_t(vb));
                    // apply_scale_32's value-range REQUIRE of the last RESCALE
                    // (q[18] = -2^min(s - 1, 31)).
                    res_bad = __builtin_amdgcn_bitop3_b32(res_bad, uint32_t(med3(sum, q[18], ~q[18])),
                                                          uint32_t(sum), 0xf6);
                    v[i] = med3(res_apply(sum, q[12], q[13], rpo, rno), E.rclo, E.rchi);
                }
            }
            if constexpr (OB == 1) {
                res[tn][tm] = pack4_u8(v[0], v[1], v[2], v[3]);
            } else if constexpr (OB == 2) {
                res[tn][2 * tm] = (uint32_t(v[0]) & 0xFFFF) | (uint32_t(v[1]) << 16);
                res[tn][2 * tm + 1] = (uint32_t(v[2]) & 0xFFFF) | (uint32_t(v[3]) << 16);
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    res[tn][4 * tm + i] = uint32_t(v[i]);
            }
            // Materialise the packed words here: otherwise the 64-bit
            // intermediates are sunk towards the final stores and held in
            // registers across every group.
#pragma unroll
            for (int w = 0; w < OB; w++)
                asm volatile("" : "+v"(res[tn][tm * OB + w]));
            if constexpr (RS && RC)
                asm volatile("" : "+v"(bad_bits));
        }
    }
    };
    if (!RS || E.one_round)
        groups(std::true_type{});
    else
        groups(std::false_type{});

    if constexpr (CS != 4) {
        // Each channel group on its own: 4 channels, OB words.
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            const int m = pixel(wave_p0 + 16 * tn + j16);
            if (m < 0)
                continue;
#pragma unroll
            for (int tm = 0; tm < TM; tm++) {
                const int cb = c0 + CS * tm;
                uint8_t* dst = E.out + (int64_t(m) * E.N + cb) * OB;
                if (cb + 4 <= E.N && (reinterpret_cast<uintptr_t>(dst) % (4 * OB)) == 0) {
                    if constexpr (OB == 1)
                        *reinterpret_cast<uint32_t*>(dst) = res[tn][tm];
                    else if constexpr (OB == 2)
                        *reinterpret_cast<v2u*>(dst) = v2u{res[tn][2 * tm], res[tn][2 * tm + 1]};
                    else
                        *reinterpret_cast<v4u*>(dst) =
                            v4u{res[tn][4 * tm], res[tn][4 * tm + 1], res[tn][4 * tm + 2], res[tn][4 * tm + 3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if (cb + e >= E.N)
                            continue;
                        const uint32_t word = res[tn][(4 * tm + e) * OB / 4];
                        const int sh = 8 * (((4 * tm + e) * OB) % 4);
                        if constexpr (OB == 1)
                            dst[e] = uint8_t(word >> sh);
                        else if constexpr (OB == 2)
                            reinterpret_cast<uint16_t*>(dst)[e] = uint16_t(word >> sh);
                        else
                            reinterpret_cast<uint32_t*>(dst)[e] = word;
                    }
                }
            }
        }
        if (bad_bits | res_bad)
            atomicOr(E.err, DERR_SCALE_RANGE);
        return;
    }
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int m = pixel(wave_p0 + 16 * tn + j16);
        if (m < 0)
            continue;
        const int64_t o = int64_t(m) * E.N + c0;
        uint8_t* dst = E.out + o * OB;
        constexpr int VB = 4 * WORDS;  // bytes this lane holds for the pixel
        if (c0 + 4 * TM <= E.N && (reinterpret_cast<uintptr_t>(dst) % (VB < 16 ? VB : 16)) == 0) {
            if constexpr (WORDS % 4 == 0) {
#pragma unroll
                for (int w = 0; w < WORDS; w += 4)
                    *reinterpret_cast<v4u*>(dst + 4 * w) =
                        v4u{res[tn][w], res[tn][w + 1], res[tn][w + 2], res[tn][w + 3]};
            } else if constexpr (WORDS == 2) {
                *reinterpret_cast<v2u*>(dst) = v2u{res[tn][0], res[tn][1]};
            } else {
                *reinterpret_cast<uint32_t*>(dst) = res[tn][0];
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4 * TM; e++) {
                if (c0 + e >= E.N)
                    continue;
                const uint32_t word = res[tn][(e * OB) / 4];
                const int sh = 8 * ((e * OB) % 4);
                if constexpr (OB == 1)
                    dst[e] = uint8_t(word >> sh);
                else if constexpr (OB == 2)
                    reinterpret_cast<uint16_t*>(dst)[e] = uint16_t(word >> sh);
                else
                    reinterpret_cast<uint32_t*>(dst)[e] = word;
            }
        }
    }
    if (bad_bits | res_bad)
        atomicOr(E.err, DERR_SCALE_RANGE);
}

// BC x BP tile, WC x WP waves, KC bytes of K per stage. PW: 1x1 stride-1
// unpadded convolution (a plain GEMM over the NHWC rows; K may be any
// multiple of 16). OB: output bytes (1, 2, 4). RS: RESCALE epilogue (else
// int32 + bias). ZW: weight zero point is nonzero.
template <int BC, int BP, int WC, int WP, int KC, bool PW, int OB, bool RS, bool ZW, bool RES = false>
__global__ void __launch_bounds__(256, 2) conv_i8_kernel(ConvI8Args Ain)
{
    ConvI8Args A = Ain;
    if constexpr (PW) {
        const int z = blockIdx.z;
        A.x += z * A.bsx;
        A.w += z * A.bsw;
        A.tab += z * A.bst;
        A.E.out += z * A.bso;
    }
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

    // The tile's epilogue table, staged in LDS behind the stage buffers
    // (with RES, the residual constants behind it).
    v4i* const s_tab = reinterpret_cast<v4i*>(smem + 2 * (BC + BP) * KC);
    for (int i = tid; i < 2 * BC; i += 256) {
        const int c = n0 + (i >> 1);
        s_tab[i] = A.tab[2 * (c < A.N ? c : A.N - 1) + (i & 1)];
    }
    int32_t* const s_res = reinterpret_cast<int32_t*>(s_tab + 2 * BC);
    if constexpr (RES) {
        for (int i = tid; i < CONV_I8_RES_WORDS * BC; i += 256) {
            const int c = n0 + i / CONV_I8_RES_WORDS;
            s_res[i] = A.rtab[(c < A.N ? c : A.N - 1) * CONV_I8_RES_WORDS + i % CONV_I8_RES_WORDS];
        }
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
    // A wave whose channels all lie past N (the last channel tile of a
    // layer whose channel count is not a multiple of the tile) only helps
    // to stage: no MFMAs, no epilogue.
    const bool wave_live = n0 + wave_c0 < A.N;
    for (int s = 0; s < nst; s++) {
        const int buf = s & 1;
        if (s + 1 < nst) {
            load((s + 1) * KC, ky, kx, ic0);
            advance();
        }
        const uint8_t* a = sA + buf * BC * KC;
        const uint8_t* b = sB + buf * BP * KC;
#pragma unroll
        for (int ks = 0; ks < (wave_live ? KC / 64 : 0); ks++) {
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
    if (wave_live) {
        auto pixel = [&](int p) { return m0 + p < A.M ? m0 + p : -1; };
        if (!RS || A.E.range)
            epilogue<TM, TN, OB, RS, ZW, true, RES>(acc, s_tab, s_rowsum, wave_c0 + grp * 4 * TM, n0, wave_p0, j16,
                                                    A.E, pixel, s_res);
        else
            epilogue<TM, TN, OB, RS, ZW, false, RES>(acc, s_tab, s_rowsum, wave_c0 + grp * 4 * TM, n0, wave_p0, j16,
                                                     A.E, pixel, s_res);
    }
}

// A direct 16-byte global->LDS load (global_load_lds_dwordx4: lane l writes
// LDS byte address `l` + 16 l, `l` wave-uniform). Issued through inline
// assembly: LLVM's wait-count pass counts a builtin LDS DMA in flight as an
// out-of-order LDS event and then makes every LDS read wait for all earlier
// ones (lgkmcnt(0)), which serialises the fragment prefetch. The callers wait
// for these loads themselves (s_waitcnt vmcnt(0) and a barrier) before
// reading what they fill.
__device__ __forceinline__ void dma16(const void* g, const void* l)
{
    const uint32_t la = __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>((const lvoid*)l)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(la) : "memory", "m0");
}

typedef __attribute__((address_space(3))) v2i lv2i;
// Transposing 8-byte LDS read: in each group of 16 lanes, lane i receives
// byte i % 8 of the 8-byte pieces addressed by lanes 2 j + i / 8 (j = 0..7),
// as byte j.
__device__ __forceinline__ v2i ldtr8(const uint8_t* p)
{
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lv2i*)((const lvoid*)p));
}

// ---------------------------------------------------------------------------
// Batched int8 MATMUL with B in its own [C][W] layout
// ---------------------------------------------------------------------------
// D[h][w] = sum_c (a[h][c] - za)(b[c][w] - zb) for every batch, in one
// kernel, on the v_mfma_i32_16x16x64_i8 tiling of conv_i8_kernel (columns w
// = its channels, rows h = its pixels): 128 columns x 32 WP rows per
// workgroup, 2 x WP waves of 64 x 32. Both operands go to LDS with direct
// global->LDS loads (wave-uniform base, per-lane 32-bit offsets), 128-byte K
// stages in a ring of three buffers with the loads of two in flight; the
// ring is unrolled so that every LDS address is a register plus an
// immediate.
// * A stage: 1 KB block (rb, ks) holds rows 16 rb .. 16 rb + 15, bytes
//   64 ks .. 64 ks + 63, lane l = 16 g + j of the block holding row 16 rb + j,
//   bytes 64 ks + 16 g .. + 15: a 16-row fragment is one contiguous read.
// * B stage: B's rows as they lie (row k = 128 bytes of columns, 8-byte
//   piece p stored at p ^ bsw(k)); a column fragment is read with
//   ds_read_b64_tr_b8: lane t of a 16-lane group addresses row kb + t / 2,
//   columns c0 + 8 (t % 2) .. + 7, so lane i receives column c0 + i of rows
//   kb .. kb + 7. The swizzle puts the 16 rows and two pieces that a half
//   wave reads in distinct banks.
// The zero-point terms: -za sum_c b[c][w] from one more MFMA per column
// fragment, against a fragment of za bytes, and -zb sum_c a[h][c] from one
// more MFMA per row fragment, with a fragment of zb bytes; both results have
// the accumulators' layout and are subtracted from them. The table holds the
// additive constant K za zb and the RESCALE parameters, independent of B's
// values. Lane (g, j) of a wave ends with the channels 16 tm + 4 g + i of its
// columns, which the shared epilogue stores group by group.
struct MatmulI8Args {
    const int8_t* a;  // [batch][H][C]
    const int8_t* b;  // [batch][C][W]
    const v4i* tab;   // [W][2] entries without column sums
    int32_t H, C, W;
    int32_t HT, WT, batch;  // row tiles, column tiles, batches
    int32_t zp_a;
    EpiArgs E;  // out [batch][H][W]; E.zp_w is B's zero point
};

// 128 columns x 32 WP rows per workgroup of 2 x WP waves; a ring of three
// stages (a ring of four measured no faster at 128 rows).
constexpr int MM_BW = 128, MM_KC = 128;  // columns, K bytes per stage
constexpr int mm_bh(int wp) { return 32 * wp; }
constexpr int mm_ns(int) { return 3; }
constexpr int mm_stage(int wp) { return (MM_BW + mm_bh(wp)) * MM_KC; }
constexpr size_t mm_lds(int wp)
{
    return size_t(mm_ns(wp)) * mm_stage(wp) + 2 * MM_BW * 16;
}

// dma16 with a wave-uniform 64-bit base and a 32-bit per-lane offset (the
// saddr form): per-stage address steps are then scalar adds.
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, const void* l)
{
    const uint32_t la = __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>((const lvoid*)l)));
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(base), "s"(la)
                 : "memory", "m0");
}

template <int WP, int OB, bool RS, bool ZA, bool ZB, bool RC>
__global__ void __launch_bounds__(128 * WP, 4 / WP) matmul_i8_kernel(MatmulI8Args A)
{
    constexpr int BW = MM_BW, BH = mm_bh(WP), KC = MM_KC, NS = mm_ns(WP), STAGE = mm_stage(WP);
    constexpr int WC = 2, NW = WC * WP;  // waves
    constexpr int TM = BW / WC / 16, TN = BH / WP / 16;
    constexpr int SA = BH * KC;               // A bytes per stage
    constexpr int NA = BH * KC / 1024 / NW;   // A direct loads per stage and wave
    constexpr int NB = BW * KC / 1024 / NW;   // B direct loads per stage and wave
    constexpr int LPS = NA + NB;
    static_assert((WP == 2 || WP == 4) && TM == 4 && TN == 2 && NA == 2, "tiling");
    // 8-byte piece p of B row k sits at p ^ bsw(k): even, so 16-byte pairs
    // stay pairs.
    auto bsw = [](int k) { return 2 * (((k >> 1) & 3) | (((k >> 4) & 1) << 2)); };

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    v4i* const s_tab = reinterpret_cast<v4i*>(smem + NS * STAGE);  // [BW][2]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave_c0 = (wave / WP) * (BW / WC);
    const int wave_p0 = (wave % WP) * (BH / WP);
    const int j16 = lane & 15;
    const int grp = lane >> 4;
    // Tile t of XCD x is workgroup x + 8 t (workgroups are dealt round-robin
    // to the XCDs), tiles ordered batch, row tile, column tile: an XCD's
    // workgroups share whole batches of A and B in its L2.
    const int ntiles = A.HT * A.WT * A.batch;
    const int tile = (ntiles & 7) == 0 ? (blockIdx.x & 7) * (ntiles >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int wt = tile % A.WT, ht = (tile / A.WT) % A.HT;
    const int h0 = ht * BH, w0 = wt * BW;
    const int64_t bz = tile / (A.WT * A.HT);
    const int8_t* const a = A.a + bz * A.H * A.C;
    const int8_t* const b = A.b + bz * A.C * A.W;

    // This thread's table entry (threads below 2 BW), stored to LDS after the
    // main loop.
    const int tcol = w0 + ((tid >> 1) & (BW - 1));
    const v4i tv = A.tab[2 * (tcol < A.W ? tcol : A.W - 1) + (tid & 1)];

    // Per-lane offsets of the direct loads from the stage's first byte of A
    // (column k0) and of B (row k0). A rows past H re-read row H - 1; B pieces
    // past W re-read the last 16 columns (neither is stored).
    uint32_t aoff[NA], boff[NB];
#pragma unroll
    for (int i = 0; i < NA; i++) {
        const int q = wave + NW * i;  // A block: rows 16 (q / 2) .., bytes 64 (q % 2) ..
        const int r = h0 + 16 * (q >> 1) + j16;
        aoff[i] = uint32_t(r < A.H ? r : A.H - 1) * uint32_t(A.C) + 16 * grp + 64 * (q & 1);
    }
#pragma unroll
    for (int i = 0; i < NB; i++) {
        const int q = wave + NW * i;  // B rows 8 q .. 8 q + 7
        const int k = 8 * q + (lane >> 3);
        const int col = w0 + 8 * ((2 * (lane & 7)) ^ bsw(k));
        boff[i] = uint32_t(k) * uint32_t(A.W) + uint32_t(col + 16 <= A.W ? col : A.W - 16);
    }
    auto issue = [&](int st, auto bufc) {
        constexpr int BUF = decltype(bufc)::value;
        uint8_t* const dst = smem + BUF * STAGE;
        const int8_t* const ab = a + st * KC;
        const int8_t* const bb = b + int64_t(st * KC) * A.W;
#pragma unroll
        for (int i = 0; i < NA; i++)
            dma16s(ab, aoff[i], dst + (wave + NW * i) * 1024);
#pragma unroll
        for (int i = 0; i < NB; i++)
            dma16s(bb, boff[i], dst + SA + (wave + NW * i) * 1024);
    };

    // LDS read offsets within a stage: B column fragments (rows 64 ks + 8 half
    // further on, where the swizzle is the same), A row fragments (ks blocks
    // 1 KB further on).
    uint32_t troff[TM], aroff[TN];
#pragma unroll
    for (int lt = 0; lt < TM; lt++) {
        const int p = ((wave_c0 + 16 * lt) >> 3) + (j16 & 1);
        const int k = 16 * grp + (j16 >> 1);
        troff[lt] = uint32_t(SA + k * BW + ((p ^ bsw(k)) << 3));
    }
#pragma unroll
    for (int lt = 0; lt < TN; lt++)
        aroff[lt] = uint32_t((((wave_p0 >> 4) + lt) * 2 * 64 + lane) * 16);

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            acc[i][j] = v4i{0, 0, 0, 0};
    // za sum_k b[k][w] for the channels of acc[tm][.] (ZA) and zb sum_k a[h][k]
    // for the rows of acc[.][tn] (ZB): the MFMAs of the column fragments with
    // a fragment of za bytes, and of a fragment of zb bytes with the row
    // fragments, leave them in acc's layout.
    v4i zcs[ZA ? TM : 1], zrs[ZB ? TN : 1];
#pragma unroll
    for (int i = 0; i < (ZA ? TM : 1); i++)
        zcs[i] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < (ZB ? TN : 1); i++)
        zrs[i] = v4i{0, 0, 0, 0};
    const int32_t za4 = int32_t(uint32_t(A.zp_a & 0xff) * 0x01010101u);
    const int32_t zb4 = int32_t(uint32_t(A.E.zp_w & 0xff) * 0x01010101u);
    const v4i zaf = v4i{za4, za4, za4, za4}, zbf = v4i{zb4, zb4, zb4, zb4};

    auto compute = [&](auto bufc) {
        constexpr int BUF = decltype(bufc)::value;
        const uint8_t* const sbase = smem + BUF * STAGE;
#pragma unroll
        for (int ks = 0; ks < KC / 64; ks++) {
            v4i af[TM], bf[TN];
#pragma unroll
            for (int lt = 0; lt < TM; lt++) {
                const v2i h0v = ldtr8(sbase + troff[lt] + (64 * ks) * BW);
                const v2i h1v = ldtr8(sbase + troff[lt] + (64 * ks + 8) * BW);
                af[lt] = v4i{h0v.x, h0v.y, h1v.x, h1v.y};
            }
#pragma unroll
            for (int lt = 0; lt < TN; lt++)
                bf[lt] = *reinterpret_cast<const v4i*>(sbase + aroff[lt] + ks * 1024);
#pragma unroll
            for (int lt = 0; lt < TM; lt++)
#pragma unroll
                for (int ln = 0; ln < TN; ln++)
                    acc[lt][ln] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[lt], bf[ln], acc[lt][ln], 0, 0, 0);
            if constexpr (ZA) {
#pragma unroll
                for (int lt = 0; lt < TM; lt++)
                    zcs[lt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[lt], zaf, zcs[lt], 0, 0, 0);
            }
            if constexpr (ZB) {
#pragma unroll
                for (int ln = 0; ln < TN; ln++)
                    zrs[ln] = __builtin_amdgcn_mfma_i32_16x16x64_i8(zbf, bf[ln], zrs[ln], 0, 0, 0);
            }
        }
    };

    const int nst = A.C / KC;
    using std::integral_constant;
    // Stage st of the loop below: wait for its loads (vmcnt(N): at most N of
    // this wave's loads outstanding, those of the next stage already issued;
    // gfx9 s_waitcnt: vmcnt in bits 3-0 and 15-14, expcnt 6-4 and lgkmcnt
    // 11-8 left at their maxima), meet at the barrier (every wave's loads of
    // stage st have landed, and every wave is done with the buffer that stage
    // st + NS - 1 overwrites: stage st - 1's), issue stage st + NS - 1 and
    // compute from buffer st % NS.
    auto step = [&](int st, auto bufc) {
        constexpr int BUF = decltype(bufc)::value;
        const int later = nst - 1 - st < NS - 2 ? nst - 1 - st : NS - 2;
        if (later >= 2)
            __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * LPS));
        else if (later == 1)
            __builtin_amdgcn_s_waitcnt(0x0F70 | LPS);
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (st + NS - 1 < nst)
            issue(st + NS - 1, integral_constant<int, (BUF + NS - 1) % NS>{});
        compute(bufc);
    };
    static_assert((NS == 3 || NS == 4) && 2 * LPS < 16, "ring of three or four buffers");
    issue(0, integral_constant<int, 0>{});
    if (nst > 1)
        issue(1, integral_constant<int, 1>{});
    if constexpr (NS == 4)
        if (nst > 2)
            issue(2, integral_constant<int, 2>{});
    for (int st = 0; st < nst; st += NS) {
        step(st, integral_constant<int, 0>{});
        if (st + 1 < nst)
            step(st + 1, integral_constant<int, 1>{});
        if (st + 2 < nst)
            step(st + 2, integral_constant<int, 2>{});
        if constexpr (NS == 4)
            if (st + 3 < nst)
                step(st + 3, integral_constant<int, 3>{});
    }
    // ---- zero-point terms and table --------------------------------------
    if (tid < 2 * BW)
        s_tab[tid] = tv;
#pragma unroll
    for (int lt = 0; lt < TM; lt++)
#pragma unroll
        for (int ln = 0; ln < TN; ln++) {
            v4u v = v4u(acc[lt][ln]);
            if constexpr (ZA)
                v -= v4u(zcs[lt]);
            if constexpr (ZB)
                v -= v4u(zrs[ln]);
            acc[lt][ln] = v4i(v);
        }
    __syncthreads();  // the table is in LDS

    // Lane (g, j) holds channels 16 tm + 4 g + i of acc[tm][tn]: the epilogue
    // stores each group of four on its own.
    auto pixel = [&](int p) { return h0 + p < A.H ? int(bz * A.H + h0 + p) : -1; };
    epilogue<TM, TN, OB, RS, false, RC, false, 16>(acc, s_tab, nullptr, wave_c0 + 4 * grp, w0, wave_p0, j16, A.E,
                                                    pixel);
}

// ---------------------------------------------------------------------------
// Stride-1 convolution over a halo tile
// ---------------------------------------------------------------------------
// A workgroup computes BC output channels x R full output rows of one image
// (R * OW <= 224 pixels). The input rows those outputs read -- R + (KH-1) dy
// rows of OW + (KW-1) dx pixels, padding positions set to the input zero
// point -- are staged once in LDS (`ICC` channels at a time, each pixel row
// padded by 16 bytes so that 16 consecutive pixels fall on distinct banks).
// The B fragment of a pixel at kernel tap (ky, kx) is then a read at the
// pixel's halo position plus a uniform tap offset: no per-tap im2col
// addressing and no re-fetch of the input per tap. Weights stream through
// NB LDS stages of KC bytes with direct global->LDS loads (no VGPR
// staging).
struct HaloArgs {
    const int8_t* x;
    const int8_t* w;
    const v4i* tab;
    int32_t N, K, IC, IH, IW, OH, OW, KH, KW, dy, dx, pt, pl;
    int32_t R, tiles_per_img;
    int32_t HR, HW, ICC, ICS, halo_bytes;
    FastDiv div_ow, div_hw, div_cpp;
    int32_t zp_x;
    EpiArgs E;
};

constexpr int HALO_TN = 7;                  // 16-pixel tiles per wave
constexpr int HALO_BP = 2 * HALO_TN * 16;   // pixels per workgroup tile
constexpr int NB = 4;                       // weight stage buffers
constexpr int HALO_WC = 4;                  // channel waves (x 2 pixel waves)
constexpr int HALO_NT = 64 * HALO_WC * 2;   // threads per workgroup

template <int BC, int KC, int OB, bool RS, bool ZW>
// (second launch bound: at least 2 waves per SIMD, i.e. 256 registers per lane)
__global__ void __launch_bounds__(HALO_NT, 2) conv_i8_halo_kernel(HaloArgs A)
{
    constexpr int NT = HALO_NT;            // 8 waves: 4 channel waves x 2 pixel waves
    constexpr int WC = HALO_WC;
    constexpr int TM = BC / (16 * WC);     // 16-channel tiles per wave
    constexpr int TN = HALO_TN;            // 16-pixel tiles per wave
    constexpr int BP = HALO_BP;
    constexpr int CPR = KC / 16;           // 16-byte chunks per weight row
    constexpr int WSLOTS = BC * CPR;       // 16-byte slots of one weight stage
    constexpr int NW = NT / 64;            // waves
    constexpr int WPW = WSLOTS >= NT ? WSLOTS / NT : 1;  // slots each loading lane loads per stage
    constexpr int LW = WSLOTS / (64 * WPW);              // waves that load weights
    static_assert(WSLOTS % (64 * WPW) == 0 && LW <= NW && TM >= 1 && 2 * BC <= NT, "tile shape");

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* const halo = smem;
    uint8_t* const sW = smem + A.halo_bytes;                              // [NB][BC][KC]
    v4i* const s_tab = reinterpret_cast<v4i*>(sW + NB * BC * KC);        // [2 BC]
    int32_t* const s_hsum = reinterpret_cast<int32_t*>(s_tab + 2 * BC);  // ZW: [HR HW]
    int32_t* const s_rowsum = s_hsum + A.HR * A.HW;                      // ZW: [BP]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wave_c0 = (wave >> 1) * (BC / WC);
    const int wave_p0 = (wave & 1) * (BP / 2);
    const int j16 = lane & 15;
    const int grp = lane >> 4;
    const int img = blockIdx.x / A.tiles_per_img;
    const int oy0 = (blockIdx.x - img * A.tiles_per_img) * A.R;
    const int rows = A.OH - oy0 < A.R ? A.OH - oy0 : A.R;
    const int npix = rows * A.OW;
    const int n0 = blockIdx.y * BC;

    // The tile's epilogue table, loaded straight into LDS (slot i = thread i;
    // channels past N repeat channel N-1). It is first read after the main
    // loop's barriers.
    if (wave * 64 < 2 * BC) {
        const int c = n0 + (tid >> 1);
        __builtin_amdgcn_global_load_lds((gvoid*)(A.tab + 2 * (c < A.N ? c : A.N - 1) + (tid & 1)),
                                         (lvoid*)(s_tab + wave * 64), 16, 0, 0);
    }
    if constexpr (ZW)
        for (int i = tid; i < A.HR * A.HW; i += NT)
            s_hsum[i] = 0;

    // Halo position of this lane's pixel in each pixel tile (pixels past the
    // tile's end read pixel 0; their results are not stored).
    int32_t pb[TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int p = wave_p0 + 16 * tn + j16;
        const int pp = p < npix ? p : 0;
        const int r = fdiv(pp, A.div_ow);
        const int ox = pp - r * A.OW;
        pb[tn] = (r * A.HW + ox) * A.ICS + grp * 16;
    }

    // Weight slots of this lane: slot = wave * WSLOTS/NW + 64 i + lane of the
    // stage buffer holds chunk (slot % CPR) ^ swz(row) of row slot / CPR.
    // Rows past N re-read row N-1 (their channels are never stored).
    int32_t woff[WPW];
#pragma unroll
    for (int i = 0; i < WPW; i++) {
        const int slot = (wave < LW ? wave : 0) * (64 * WPW) + 64 * i + lane;
        const int row = slot / CPR;
        const int oc = n0 + row;
        woff[i] = (oc < A.N ? oc : A.N - 1) * A.K + (((slot % CPR) ^ swz<KC>(row)) << 4);
    }
    auto dma_w = [&](int buf, int kst) {
        if (LW < NW && wave >= LW)
            return;
        const int8_t* src = A.w + kst;
        uint8_t* dst = sW + buf * (BC * KC) + wave * (64 * WPW) * 16;
#pragma unroll
        for (int i = 0; i < WPW; i++)
            __builtin_amdgcn_global_load_lds((gvoid*)(src + woff[i]), (lvoid*)(dst + 1024 * i), 16, 0, 0);
    };

    const uint32_t zf = uint32_t(uint8_t(A.zp_x)) * 0x01010101u;
    const v4u zfill = v4u{zf, zf, zf, zf};
    // Stage ICC channels of the halo; loads are issued in batches of U so
    // their latencies overlap.
    auto fill_halo = [&](int icc0) {
        constexpr int U = 8;
        const int cpp = A.ICC >> 4;
        const int total = A.HR * A.HW * cpp;
        const int8_t* xi = A.x + img * A.IH * A.IW * A.IC + icc0;
        for (int q0 = 0; q0 < total; q0 += NT * U) {
            v4u v[U];
            int32_t dst[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int q = q0 + NT * u + tid;
                const int qq = q < total ? q : 0;
                const int hp = fdiv(qq, A.div_cpp);
                const int c = qq - hp * cpp;
                const int hr = fdiv(hp, A.div_hw);
                const int hc = hp - hr * A.HW;
                const int iy = oy0 - A.pt + hr;
                const int ix = hc - A.pl;
                const bool ok = unsigned(iy) < unsigned(A.IH) && unsigned(ix) < unsigned(A.IW);
                const v4u t = ld16(xi + (ok ? (iy * A.IW + ix) * A.IC + c * 16 : 0));
                v[u] = ok ? t : zfill;
                dst[u] = q < total ? hp * A.ICS + c * 16 : -1;
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (dst[u] >= 0)
                    *reinterpret_cast<v4u*>(halo + dst[u]) = v[u];
        }
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
            acc[a][b] = v4i{0, 0, 0, 0};

    // Software pipeline over the stages of a halo pass: the weights of stages
    // s+2 and s+3 are in flight (direct loads into buffer (s+j) % NB) and the
    // A/B fragments of stage s+1 are read from LDS while stage s's MFMAs run,
    // so each stage starts its MFMAs right after the barrier.
    constexpr int KS = KC / 64;
    const int subs = A.ICC / KC;
    const int nst = A.KH * A.KW * subs;
    v4i fa0[KS][TM], fb0[KS][TN], fa1[KS][TM], fb1[KS][TN];
    for (int icc0 = 0; icc0 < A.IC; icc0 += A.ICC) {
        if (icc0 > 0)
            __syncthreads();  // the previous pass has finished reading halo and weights
        // Stage coordinates (tap ky, kx and KC-chunk `sub`) of the next DMA
        // and of the next fragment load.
        int dky = 0, dkx = 0, dsub = 0, lky = 0, lkx = 0, lsub = 0;
        auto next = [&](int& ky, int& kx, int& sub) {
            if (++sub == subs) {
                sub = 0;
                if (++kx == A.KW) {
                    kx = 0;
                    ky++;
                }
            }
        };
        auto kstage = [&](int ky, int kx, int sub) { return (ky * A.KW + kx) * A.IC + icc0 + sub * KC; };
        auto load_frags = [&](v4i(&fa)[KS][TM], v4i(&fb)[KS][TN], int buf, int ky, int kx, int sub) {
            const uint8_t* hb = halo + (ky * A.dy * A.HW + kx * A.dx) * A.ICS + sub * KC;
            const uint8_t* wb = sW + buf * (BC * KC);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
#pragma unroll
                for (int tm = 0; tm < TM; tm++) {
                    const int row = wave_c0 + (j16 >> 2) * (4 * TM) + 4 * tm + (j16 & 3);
                    fa[ks][tm] =
                        *reinterpret_cast<const v4i*>(wb + row * KC + (((ks * 4 + grp) ^ swz<KC>(row)) << 4));
                }
#pragma unroll
                for (int tn = 0; tn < TN; tn++)
                    fb[ks][tn] = *reinterpret_cast<const v4i*>(hb + pb[tn] + ks * 64);
            }
        };
        auto mfmas = [&](const v4i(&fa)[KS][TM], const v4i(&fb)[KS][TN]) {
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
#pragma unroll
                for (int tm = 0; tm < TM; tm++)
#pragma unroll
                    for (int tn = 0; tn < TN; tn++)
                        acc[tm][tn] =
                            __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[ks][tm], fb[ks][tn], acc[tm][tn], 0, 0, 0);
        };

        // The first weight stages go out before the halo loads so that their
        // latencies overlap.
        for (int b = 0; b < NB - 1 && b < nst; b++) {
            dma_w(b, kstage(dky, dkx, dsub));
            next(dky, dkx, dsub);
        }
        fill_halo(icc0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if constexpr (ZW) {
            const int cpp = A.ICC >> 4;
            for (int hp = tid; hp < A.HR * A.HW; hp += NT) {
                int32_t t = 0;
                for (int c = 0; c < cpp; c++) {
                    const v4u v = *reinterpret_cast<const v4u*>(halo + hp * A.ICS + c * 16);
                    t = __builtin_amdgcn_sdot4(int(v.x), 0x01010101, t, false);
                    t = __builtin_amdgcn_sdot4(int(v.y), 0x01010101, t, false);
                    t = __builtin_amdgcn_sdot4(int(v.z), 0x01010101, t, false);
                    t = __builtin_amdgcn_sdot4(int(v.w), 0x01010101, t, false);
                }
                s_hsum[hp] += t;
            }
        }
        load_frags(fa0, fb0, 0, lky, lkx, lsub);
        next(lky, lkx, lsub);
        // Buffers of the next DMA and the next fragment load.
        int dbuf = NB - 1, lbuf = 1;
        auto stage = [&](int s, v4i(&ca)[KS][TM], v4i(&cb)[KS][TN], v4i(&na)[KS][TM], v4i(&nb)[KS][TN]) {
            const bool more = s + NB - 1 < nst;
            if (more) {
                dma_w(dbuf, kstage(dky, dkx, dsub));
                next(dky, dkx, dsub);
                dbuf = dbuf == NB - 1 ? 0 : dbuf + 1;
            }
            if (s + 1 < nst) {
                load_frags(na, nb, lbuf, lky, lkx, lsub);
                next(lky, lkx, lsub);
                lbuf = lbuf == NB - 1 ? 0 : lbuf + 1;
            }
            mfmas(ca, cb);
            // The fragments of s+1 and this wave's weight loads of s+2 have
            // landed; the loads of s+3 issued above (WPW per lane) may still
            // be in flight (vmcnt in bits 3:0, expcnt 7 = no wait, lgkmcnt 0).
            if (more)
                __builtin_amdgcn_s_waitcnt(0x70 | WPW);
            else
                __builtin_amdgcn_s_waitcnt(0x70);
            __syncthreads();
        };
        for (int s = 0; s < nst; s += 2) {
            stage(s, fa0, fb0, fa1, fb1);
            if (s + 1 < nst)
                stage(s + 1, fa1, fb1, fa0, fb0);
        }
    }

    if constexpr (ZW) {
        for (int p = tid; p < BP; p += NT) {
            int32_t t = 0;
            if (p < npix) {
                const int r = fdiv(p, A.div_ow);
                const int ox = p - r * A.OW;
                for (int ky2 = 0; ky2 < A.KH; ky2++)
                    for (int kx2 = 0; kx2 < A.KW; kx2++)
                        t += s_hsum[(r + ky2 * A.dy) * A.HW + ox + kx2 * A.dx];
            }
            s_rowsum[p] = t;
        }
        __syncthreads();
    }

    const int m0 = (img * A.OH + oy0) * A.OW;
    auto pixel = [&](int p) { return p < npix ? m0 + p : -1; };
    if (!RS || A.E.range)
        epilogue<TM, TN, OB, RS, ZW, true>(acc, s_tab, s_rowsum, wave_c0 + grp * 4 * TM, n0, wave_p0, j16, A.E, pixel);
    else
        epilogue<TM, TN, OB, RS, ZW, false>(acc, s_tab, s_rowsum, wave_c0 + grp * 4 * TM, n0, wave_p0, j16, A.E,
                                            pixel);
}

// ---------------------------------------------------------------------------
// Stride-1 convolution on v_mfma_i32_32x32x32_i8 with the input halo and the
// weights streamed through LDS.
//
// A workgroup computes BC output channels x up to 256 consecutive output
// pixels of one image (R whole output rows) with BC / 16 waves: wave w owns
// channels 64 (w / 4) .. + 63 (two 32-channel tiles) of the 32-pixel tiles
// w % 4 and w % 4 + 4, so one weight fragment feeds two MFMAs and so does
// one pixel fragment. Two waves per SIMD (BC = 128) keep each wave's LDS
// reads (4 KB per tap) within what one wave can draw from LDS while the
// SIMD's MFMAs run back to back.
//
// K is walked as (32-channel pass, tap). The halo (R + (KH-1) dy rows of
// OW + (KW-1) dx positions) is staged 64 input channels at a time in a ring
// of two LDS buffers, each position's 64 bytes loaded by 4 lanes; the
// weights of a pass (every tap) sit in one of two LDS buffers. While a pass
// is multiplied, the next pass's weights (and, at the first pass of a
// stage, the next stage's halo) are fetched by direct global->LDS loads.
// The weights come pre-packed in exactly their LDS image
// ([block][pass][tap][channel tile][lane][16 bytes]), so each of those loads
// reads 1 KB of contiguous memory.
//
// MFMA operand layout (checked on the device): lane l supplies row l % 32 of
// A and column l % 32 of B, both with the 16 bytes of k-half l / 32; result
// element i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.
// A = weights, B = pixels. Weight rows are permuted, row r <- channel
// 16 ((r >> 2) & 1) + 4 (r >> 3) + (r & 3), so that result element i of lane
// l is channel 16 (l / 32) + i: each lane ends with 16 consecutive channels
// of one pixel per tile, stored as one vector. The accumulators start at the
// channel's additive constant (bias and zero-point terms).
//
// Halo stage layout: [position hp][4 chunks of 16 bytes], chunk c stored at
// c ^ ((hp >> 2) & 3), so that 16 consecutive positions reading one logical
// chunk hit 16 distinct bank groups. Padding taps (and channels past IC in
// a 32-channel last stage) are loaded from 16 bytes of the input zero point
// stored after the table.
// ---------------------------------------------------------------------------
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

// Element type of the halo kernel's operands: int8 (the table-driven
// epilogue), or bf16 / fp16 with fp32 accumulation (the float epilogue
// round(round(acc) + bias) of src/ops/conv.rs:493-495). The kernel works on
// bytes: a float pass covers 16 channels (32 bytes), as an int8 pass covers
// 32.
enum HaloElem : int { HE_I8 = 0, HE_BF16 = 1, HE_F16 = 2 };

struct Halo32Args {
    const int8_t* x;
    const int8_t* wp;  // packed weights
    const v4i* tab;    // [N][2] entries, 16 bytes of the input zero point, [N] additive constants
    int32_t N, IC, IH, IW, OH, OW, KW, taps, dy, dx, pt, pl;
    int32_t R, tiles_per_img, HR, HW;
    int32_t PG, TB, KP;  // waves along the pixels, 32-pixel tiles per wave, units per pass: the launch's template
    int32_t sbytes;  // LDS bytes of one halo stage (HR*HW*64, 1 KB multiple)
    int32_t wbytes;  // bytes of one pass's weights (taps * BC * 32)
    FastDiv div_ow, div_hw;
    EpiArgs E;          // int8: the table epilogue; float: out, N
    const int8_t* zfill;  // 16 bytes loaded for padding taps: the input zero point (int8), zeros (float)
    const float* fbias;   // float: per-channel bias as f32 values (or null)
    int32_t fbias_len, fmt;
};

// Pixel slots of a workgroup with PG waves along the pixels, TB 32-pixel
// tiles each.
constexpr int h32_bp(int pg, int tb) { return pg * 32 * tb; }
constexpr int H32_BP_MAX = h32_bp(8, 2);

// Weight row of MFMA row r (see above).
__device__ __forceinline__ int h32_row_channel(int r) { return 16 * ((r >> 2) & 1) + 4 * (r >> 3) + (r & 3); }

// One 32x32 MFMA step of the halo kernel: 16 bytes of A and B per lane (32
// int8 or 16 bf16 / fp16 reduction elements).
template <int EL, typename Acc>
__device__ __forceinline__ Acc h32_mfma(const v4i& a, const v4i& b, const Acc& c)
{
    if constexpr (EL == HE_I8)
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
    else if constexpr (EL == HE_BF16)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0,
                                                       0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0,
                                                      0);
}

// Float epilogue of the 32x32 layout (lane (h, l32) holds channels
// 32 a + 16 h + 0..15 of tile pixel 32 (pw + PG b) + l32):
// out = round(round(acc) + bias) in the output format, or acc for fp32
// output without bias (src/ops/conv.rs:493-495). OB: output bytes (4 fp32,
// 2 bf16 / fp16).
template <int TA, int TB, int PG, int OB, typename PixelMap>
__device__ __forceinline__ void epilogue32f(v16f (&acc)[TA][TB], int n0, int pw, int lane, const Halo32Args& A,
                                            PixelMap pixel)
{
    const int l32 = lane & 31, h = lane >> 5;
#pragma unroll
    for (int b = 0; b < TB; b++) {
        const int64_t m = pixel(32 * (pw + PG * b) + l32);
        if (m < 0)
            continue;
#pragma unroll
        for (int a = 0; a < TA; a++) {
            const int c0 = n0 + 32 * a + 16 * h;
            if (c0 >= A.E.N)
                continue;
            uint32_t res[4 * OB];
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int c = c0 + i < A.E.N ? c0 + i : A.E.N - 1;
                float r = acc[a][b][i];
                if (A.fbias)  // the file builds with -ffp-contract=off: no fused bias add
                    r = round_fmt16(round_fmt16(r, A.fmt) + A.fbias[A.fbias_len == 1 ? 0 : c], A.fmt);
                if constexpr (OB == 4) {
                    res[i] = __builtin_bit_cast(uint32_t, r);
                } else {
                    const uint32_t bits = A.fmt == FMT_F16 ? f32_to_f16_bits(r) : f32_to_bf16_bits(r);
                    res[i / 2] = (i & 1) ? (res[i / 2] | (bits << 16)) : bits;
                }
            }
            uint8_t* dst = A.E.out + (m * A.E.N + c0) * OB;
            if (c0 + 16 <= A.E.N && ((m * A.E.N + c0) * OB) % 16 == 0) {
#pragma unroll
                for (int wd = 0; wd < 4 * OB; wd += 4)
                    *reinterpret_cast<v4u*>(dst + 4 * wd) = v4u{res[wd], res[wd + 1], res[wd + 2], res[wd + 3]};
            } else {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    if (c0 + e >= A.E.N)
                        continue;
                    if constexpr (OB == 4)
                        reinterpret_cast<uint32_t*>(dst)[e] = res[e];
                    else
                        reinterpret_cast<uint16_t*>(dst)[e] = uint16_t(res[e / 2] >> (16 * (e & 1)));
                }
            }
        }
    }
}

// Epilogue of the 32x32 layout: lane (h, l32) holds channels 32 a + 16 h +
// 0..15 (counted from n0; s_tab starts at channel n0) of tile pixel
// 32 (pw + PG b) + l32 in acc[a][b], the channel's additive constant already
// included.
template <int TA, int TB, int PG, int OB, bool RS, bool ZW, typename PixelMap>
__device__ __forceinline__ void epilogue32(v16i (&acc)[TA][TB], const v4i* s_tab, const int32_t* s_rowsum, int n0,
                                           int pw, int lane, const EpiArgs& E, PixelMap pixel)
{
    const int l32 = lane & 31, h = lane >> 5;
    // Nonzero when a value fails apply_scale_32's range REQUIRE (VALU
    // accumulation: one bitwise op per value, no scalar round trips).
    uint32_t bad_bits = 0;
    int32_t zwx[TB];
    int64_t m[TB];
#pragma unroll
    for (int b = 0; b < TB; b++) {
        const int p = 32 * (pw + PG * b) + l32;
        m[b] = pixel(p);
        zwx[b] = 0;
        if constexpr (ZW)
            zwx[b] = int32_t(uint32_t(E.zp_w) * uint32_t(s_rowsum[p]));
    }
    // Table entries of the lane's channels, one group of 4 at a time, read
    // a group ahead of the arithmetic that uses them.
    auto ld_tab = [&](int grp, v4i(&t0)[4], v4i(&t1)[4]) {
        const int cl = 32 * (grp >> 2) + 16 * h + 4 * (grp & 3);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            t0[i] = s_tab[2 * (cl + i)];
            if constexpr (RS)
                t1[i] = s_tab[2 * (cl + i) + 1];
        }
    };
    // RC: apply_scale_32's value-range REQUIRE is checked (some channel's
    // shift is below 32 and the table could not rule a failure out).
    auto body = [&](auto rc) {
        constexpr bool RC = RS && decltype(rc)::value;
        v4i tn0[4], tn1[4];
        ld_tab(0, tn0, tn1);
#pragma unroll
        for (int a = 0; a < TA; a++) {
            const int cl = 32 * a + 16 * h;  // tile channel of element 0
            uint32_t res[TB][4 * OB];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                __builtin_amdgcn_sched_barrier(0);
                v4i t0[4], t1[4];
                int32_t hi[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    t0[i] = tn0[i];
                    t1[i] = tn1[i];
                    if constexpr (RC)
                        hi[i] = ~t0[i].z;
                }
                if (4 * a + g + 1 < 4 * TA)
                    ld_tab(4 * a + g + 1, tn0, tn1);
#pragma unroll
                for (int b = 0; b < TB; b++) {
                    int32_t v[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int32_t x = int32_t(uint32_t(acc[a][b][4 * g + i]) - uint32_t(zwx[b]));
                        if constexpr (RS) {
                            // Same arithmetic as epilogue(): range REQUIRE of
                            // apply_scale_32, 64-bit scale with the per-sign
                            // rounding constant, output zero point and clamp.
                            if constexpr (RC)
                                bad_bits = __builtin_amdgcn_bitop3_b32(bad_bits, uint32_t(med3(x, t0[i].z, hi[i])),
                                                                       uint32_t(x), 0xf6);  // bad | (med3 ^ x)
                            const int64_t rp = __builtin_bit_cast(int64_t, v2i{t1[i].x, t1[i].y});
                            const int64_t rn = __builtin_bit_cast(int64_t, v2i{t1[i].z, t1[i].w});
                            const int32_t r = int32_t((int64_t(x) * int64_t(t0[i].y) + (x >= 0 ? rp : rn)) >> t0[i].w);
                            v[i] = med3(r, E.clo, E.chi);  // output zero point folded into rp, rn
                        } else {
                            v[i] = x;
                        }
                    }
                    if constexpr (OB == 1) {
                        // Low bytes of v0..v3 (v_perm_b32: selector bytes 0-3
                        // pick the second operand, 4-7 the first, 0x0c zero).
                        const uint32_t p01 = __builtin_amdgcn_perm(uint32_t(v[1]), uint32_t(v[0]), 0x0c0c0400u);
                        const uint32_t p23 = __builtin_amdgcn_perm(uint32_t(v[3]), uint32_t(v[2]), 0x0c0c0400u);
                        res[b][g] = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
                    } else if constexpr (OB == 2) {
                        res[b][2 * g] = __builtin_amdgcn_perm(uint32_t(v[1]), uint32_t(v[0]), 0x05040100u);
                        res[b][2 * g + 1] = __builtin_amdgcn_perm(uint32_t(v[3]), uint32_t(v[2]), 0x05040100u);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            res[b][4 * g + i] = uint32_t(v[i]);
                    }
#pragma unroll
                    for (int wd = 0; wd < OB; wd++)
                        asm volatile("" : "+v"(res[b][g * OB + wd]));
                    // Kept as a vector value (left alone, the compiler turns the
                    // accumulation into compares and scalar ORs, a VALU -> SALU
                    // dependency per value).
                    if constexpr (RC)
                        asm volatile("" : "+v"(bad_bits));
                }
            }
            const int c0 = n0 + cl;
#pragma unroll
            for (int b = 0; b < TB; b++) {
                if (m[b] < 0)
                    continue;
                const int64_t o = m[b] * E.N + c0;
                uint8_t* dst = E.out + o * OB;
                if (c0 + 16 <= E.N && ((o * OB) & 15) == 0) {
#pragma unroll
                    for (int wd = 0; wd < 4 * OB; wd += 4)
                        *reinterpret_cast<v4u*>(dst + 4 * wd) =
                            v4u{res[b][wd], res[b][wd + 1], res[b][wd + 2], res[b][wd + 3]};
                } else {
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        if (c0 + e >= E.N)
                            continue;
                        const uint32_t word = res[b][(e * OB) / 4];
                        const int sh = 8 * ((e * OB) % 4);
                        if constexpr (OB == 1)
                            dst[e] = uint8_t(word >> sh);
                        else if constexpr (OB == 2)
                            reinterpret_cast<uint16_t*>(dst)[e] = uint16_t(word >> sh);
                        else
                            reinterpret_cast<uint32_t*>(dst)[e] = word;
                    }
                }
            }
        }
    };
    if (E.range)
        body(std::true_type{});
    else
        body(std::false_type{});
    if (bad_bits)
        atomicOr(E.err, DERR_SCALE_RANGE);
}

// KT: taps when fixed at compile time (9 = 3x3; the tap loop is then fully
// unrolled so that each tap waits only for its own fragments), 0 = any.
// PG: waves along the pixels (each wave takes 64 channels), so BC / 64 * PG
// waves in all; TB: 32-pixel tiles per wave; EL: HaloElem (the float kinds
// have no zero points, RESCALE or table); KP: 32-byte reduction units per
// pass (2: each pass covers a whole 64-byte halo stage, half the barriers and
// load bursts of KP 1, twice the weight buffer).
template <int EL, int BC, int PG, int TB, int KT, int OB, bool RS, bool ZW, int KP = 1>
__global__ void __launch_bounds__(BC / 64 * PG * 64, 2) conv_i8_halo32_kernel(Halo32Args A)
{
    static_assert(KP == 1 || KP == 2, "one or two reduction units per pass");
    static_assert(EL == HE_I8 || (!RS && !ZW), "float halo convolutions have no RESCALE or zero points");
    using Acc = std::conditional_t<EL == HE_I8, v16i, v16f>;
    constexpr int NT = BC / 64 * PG * 64;  // threads
    constexpr int TA = 2;                  // 32-channel tiles per wave
    constexpr int BP = h32_bp(PG, TB);

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* const halo = smem;                                          // [2][sbytes]
    uint8_t* const wbuf = smem + 2 * A.sbytes;                           // [2][wbytes]
    v4i* const s_tab = reinterpret_cast<v4i*>(wbuf + 2 * KP * A.wbytes);  // [2 BC]
    int32_t* const s_hsum = reinterpret_cast<int32_t*>(s_tab + 2 * BC);  // ZW: [HR HW]
    int32_t* const s_rowsum = s_hsum + A.HR * A.HW;                      // ZW: [BP]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pw = wave % PG;         // pixel tiles pw, pw + PG, ..
    const int cw = 64 * (wave / PG);  // first channel of the wave (tile-relative)
    const int l32 = lane & 31;
    const int h = lane >> 5;
    // Workgroups are dealt round-robin to the 8 XCDs (each with its own L2);
    // when their count allows, tile t of XCD x is workgroup x + 8 t, so that
    // neighbouring row tiles, which share halo rows, meet in one L2.
    const int tile = (gridDim.x & 7) == 0 ? (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int img = tile / A.tiles_per_img;
    const int oy0 = (tile - img * A.tiles_per_img) * A.R;
    const int rows = A.OH - oy0 < A.R ? A.OH - oy0 : A.R;
    const int npix = rows * A.OW;
    const int n0 = blockIdx.y * BC;
    const int hw = A.HR * A.HW;
    const int taps = KT > 0 ? KT : A.taps;
    const int passes = A.IC >> 5;  // 32-byte reduction units; the loop takes KP per pass
    const int npass = passes / KP;

    // Epilogue table straight into LDS (channels past N repeat channel N-1).
    if (EL == HE_I8 && tid < 2 * BC) {
        const int c = n0 + (tid >> 1);
        dma16(A.tab + 2 * (c < A.N ? c : A.N - 1) + (tid & 1), s_tab + wave * 64);
    }
    if constexpr (ZW)
        for (int i = tid; i < hw; i += NT)
            s_hsum[i] = 0;

    // Additive constants of this lane's channels (cw + 32 a + 16 h + i for
    // result element i), fetched now and moved into the accumulators once
    // the first loads have landed (int8; float accumulators start at 0).
    Acc acc[TA][TB], init[TA];
    if constexpr (EL != HE_I8) {
#pragma unroll
        for (int a = 0; a < TA; a++)
            init[a] = Acc{};
    } else {
        const int32_t* adds = reinterpret_cast<const int32_t*>(A.tab + 2 * A.N + 1);
#pragma unroll
        for (int a = 0; a < TA; a++) {
            const int c = n0 + cw + 32 * a + 16 * h;
            if (c + 16 <= A.N) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const v4i v = *reinterpret_cast<const v4i*>(adds + c + 4 * q);
                    init[a][4 * q] = v.x;
                    init[a][4 * q + 1] = v.y;
                    init[a][4 * q + 2] = v.z;
                    init[a][4 * q + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 16; i++)
                    init[a][i] = adds[c + i < A.N ? c + i : A.N - 1];
            }
        }
    }

    // Halo position (tap 0) of this lane's pixel in each tile; pixels past
    // the tile's end read pixel 0 and are not stored. With one tile per wave
    // (the layout for short tiles), a wave whose tile holds no pixel skips
    // its MFMAs and epilogue; its loads and barriers stay. (The branch costs
    // the two-tile layouts' tap loop more than the idle waves would save.)
    const bool live = TB > 1 || 32 * pw < npix;
    int32_t hpos[TB];
#pragma unroll
    for (int b = 0; b < TB; b++) {
        const int p = 32 * (pw + PG * b) + l32;
        const int pp = p < npix ? p : 0;
        const int r = fdiv(pp, A.div_ow);
        hpos[b] = r * A.HW + pp - r * A.OW;
    }

    const int8_t* const xi = A.x + int64_t(img) * A.IH * A.IW * A.IC;
    const int8_t* const zfill = A.zfill;
    const int8_t* const wsrc = A.wp + int64_t(blockIdx.y) * passes * A.wbytes + lane * 16;
    const int nwq = taps * (BC / 32);  // 1 KB groups of one pass's weights
    auto dma_w = [&](int pass) {
        const int8_t* src = wsrc + int64_t(pass) * KP * A.wbytes;
        uint8_t* dst = wbuf + (pass & 1) * KP * A.wbytes;
        for (int j = wave; j < KP * nwq; j += NT / 64)
            dma16(src + j * 1024, dst + j * 1024);
    };
    // Halo stage st (input channels 64 st ..): 16-byte slot s of the LDS
    // image is chunk s % 4 of position s / 4, stored swizzled; slots past the
    // image (the last group's tail) load the zero-point fill into padding.
    auto dma_halo = [&](int st) {
        const int total = hw * 4;
        const int ch0 = 64 * st;
        uint8_t* const dst = halo + (st & 1) * A.sbytes;
        for (int s0 = wave * 64; s0 < total; s0 += NT) {
            const int sl = s0 + lane;
            const int hp = sl >> 2;
            const int c = (sl & 3) ^ ((hp >> 2) & 3);
            const int hr = fdiv(hp, A.div_hw);
            const int iy = oy0 - A.pt + hr;
            const int ix = hp - hr * A.HW - A.pl;
            const bool ok = sl < total && unsigned(iy) < unsigned(A.IH) && unsigned(ix) < unsigned(A.IW) &&
                            ch0 + 16 * c < A.IC;
            dma16(ok ? xi + (iy * A.IW + ix) * A.IC + ch0 + 16 * c : zfill, dst + s0 * 16);
        }
    };

    dma_halo(0);
    dma_w(0);
    for (int pass = 0; pass < npass; pass++) {
        // The loads of this pass (issued one pass earlier, or above) have
        // landed, and every wave is done with the buffers the next loads
        // overwrite.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (pass == 0) {
#pragma unroll
            for (int a = 0; a < TA; a++)
#pragma unroll
                for (int b = 0; b < TB; b++)
                    acc[a][b] = init[a];
        }
        // Halo stage of this pass; a pass that opens a stage also loads
        // the next one.
        const int st = KP == 2 ? pass : pass >> 1;
        const bool opens = KP == 2 || (pass & 1) == 0;
        if (opens && 2 * (st + 1) < passes)
            dma_halo(st + 1);
        if (pass + 1 < npass)
            dma_w(pass + 1);
        if constexpr (ZW) {
            if (opens) {
                const uint8_t* hs = halo + (st & 1) * A.sbytes;
                for (int hp = tid; hp < hw; hp += NT) {
                    int32_t t = s_hsum[hp];
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        if (64 * st + 16 * c >= A.IC)
                            break;  // zero-point fill past the last channel
                        const v4u v = *reinterpret_cast<const v4u*>(hs + (hp * 4 + (c ^ ((hp >> 2) & 3))) * 16);
                        t = __builtin_amdgcn_sdot4(int(v.x), 0x01010101, t, false);
                        t = __builtin_amdgcn_sdot4(int(v.y), 0x01010101, t, false);
                        t = __builtin_amdgcn_sdot4(int(v.z), 0x01010101, t, false);
                        t = __builtin_amdgcn_sdot4(int(v.w), 0x01010101, t, false);
                    }
                    s_hsum[hp] = t;
                }
            }
        }
        const uint8_t* const wb = wbuf + (pass & 1) * KP * A.wbytes + lane * 16;
        const uint8_t* const hb = halo + (st & 1) * A.sbytes;
        // The fragments of tap t + 1 are read while tap t's MFMAs run. Unit
        // u of the pass: weights at u wbytes in the pass's buffer, halo
        // logical chunk 2 u + h (KP 2) or 2 (pass & 1) + h (KP 1).
        auto load = [&](v4i(&fa)[KP][TA], v4i(&fb)[KP][TB], int t, int ky, int kx) {
            const int off = ky * A.dy * A.HW + kx * A.dx;
#pragma unroll
            for (int u = 0; u < KP; u++) {
#pragma unroll
                for (int a = 0; a < TA; a++)
                    fa[u][a] = *reinterpret_cast<const v4i*>(wb + u * A.wbytes + (t * (BC / 32) + cw / 32 + a) * 1024);
                const int cl = KP == 2 ? 2 * u + h : 2 * (pass & 1) + h;
#pragma unroll
                for (int b = 0; b < TB; b++) {
                    const int hp = hpos[b] + off;
                    fb[u][b] = *reinterpret_cast<const v4i*>(hb + (hp * 4 + (cl ^ ((hp >> 2) & 3))) * 16);
                }
            }
        };
        auto mfma = [&](const v4i(&fa)[KP][TA], const v4i(&fb)[KP][TB]) {
#pragma unroll
            for (int u = 0; u < KP; u++)
#pragma unroll
                for (int b = 0; b < TB; b++)
#pragma unroll
                    for (int a = 0; a < TA; a++)
                        acc[a][b] = h32_mfma<EL>(fa[u][a], fb[u][b], acc[a][b]);
        };
        if (!live) {
            // no pixels: only the loads and barriers of the pass
        } else if constexpr (KT == 9) {
            v4i fa[2][KP][TA], fb[2][KP][TB];
            load(fa[0], fb[0], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 9; t++) {
                // Scheduling fences keep the next tap's reads ahead of this
                // tap's MFMAs (left alone, the scheduler sinks them below the
                // MFMAs to save registers, and the reads' latency shows).
                __builtin_amdgcn_sched_barrier(0);
                if (t + 1 < 9)
                    load(fa[(t + 1) & 1], fb[(t + 1) & 1], t + 1, (t + 1) / 3, (t + 1) % 3);
                __builtin_amdgcn_sched_barrier(0);
                mfma(fa[t & 1], fb[t & 1]);
            }
            __builtin_amdgcn_sched_barrier(0);
        } else {
            int ky = 0, kx = 0;
            auto step = [&]() {
                if (++kx == A.KW) {
                    kx = 0;
                    ky++;
                }
            };
            v4i fa0[KP][TA], fb0[KP][TB], fa1[KP][TA], fb1[KP][TB];
            load(fa0, fb0, 0, 0, 0);
            step();
            for (int t = 0; t < taps; t += 2) {
                const bool two = t + 1 < taps;
                if (two) {
                    load(fa1, fb1, t + 1, ky, kx);
                    step();
                }
                mfma(fa0, fb0);
                if (two) {
                    if (t + 2 < taps) {
                        load(fa0, fb0, t + 2, ky, kx);
                        step();
                    }
                    mfma(fa1, fb1);
                }
            }
        }
    }

    if constexpr (ZW) {
        __syncthreads();  // every stage's sums are in
        for (int p = tid; p < BP; p += NT) {
            int32_t t = 0;
            if (p < npix) {
                const int r = fdiv(p, A.div_ow);
                const int ox = p - r * A.OW;
                for (int t2 = 0; t2 < taps; t2++) {
                    const int ky2 = t2 / A.KW, kx2 = t2 - ky2 * A.KW;
                    t += s_hsum[(r + ky2 * A.dy) * A.HW + ox + kx2 * A.dx];
                }
            }
            s_rowsum[p] = t;
        }
        __syncthreads();
    }

    const int m0 = (img * A.OH + oy0) * A.OW;
    if (live) {
        if constexpr (EL == HE_I8)
            epilogue32<TA, TB, PG, OB, RS, ZW>(acc, s_tab + 2 * cw, s_rowsum, n0 + cw, pw, lane, A.E,
                                               [&](int p) { return p < npix ? m0 + p : -1; });
        else
            epilogue32f<TA, TB, PG, OB>(acc, n0 + cw, pw, lane, A, [&](int p) { return p < npix ? m0 + p : -1; });
    }
}

// ---------------------------------------------------------------------------
// Row-tile int8 3x3 convolution: stride 1, no dilation, output rows of 17 to
// 30 pixels, 128 input channels, no weight zero point (the ResNet-scale
// [N,28,28,128] layers). A workgroup computes 32 CB output channels x RG RW
// output rows with eight waves, two per SIMD: four producer waves issue the
// MFMAs and four consumer waves run the epilogue, so that the epilogue's
// VALU work issues beside the other wave's matrix work instead of between
// its own MFMAs.
//
// Producer wave p owns 32 channels x RW rows: one 32-pixel MFMA tile per
// output row, output pixel ox in lane ox (lanes past the row compute the
// padded positions and store nothing). For reduction chunk q (32 input
// channels) and column tap kx, the B fragment of halo row hr is the operand
// of row tap ky for output row hr - ky: one LDS read feeds up to three
// MFMAs. The wave's A fragments (the whole reduction: IC / 32 x 9 of them)
// stay in VGPRs, loaded once from the packed weights, each workgroup
// starting at its own chunk; the accumulators start at the channels'
// additive constants. Rows run in phases of 2, 2, 2 and 1; at the end of a
// phase the producer writes its accumulators to a transfer buffer in LDS
// (two buffers, alternating) and the workgroup meets at a barrier; the
// consumer wave p + 4 then turns those rows into output bytes (RESCALE,
// CLAMP, packing, stores) while its producer computes the next phase.
//
// The halo (HR rows x 32 positions x IC bytes; 16-byte chunk c of position
// pos stored at chunk c ^ ((pos >> 1) & 7), so that 16 consecutive
// positions reading one chunk hit 16 distinct bank groups) is one LDS image
// loaded by all eight waves, positions outside the image from the
// zero-point fill. Only the rows of the first phase are waited for before
// it starts; the others are loaded behind the weights and stored while it
// computes. The consumers stage the epilogue table through LDS.
// ---------------------------------------------------------------------------
struct RowsArgs {
    const int8_t* x;
    const int8_t* wp;  // packed weights, 32-channel blocks
    const v4i* tab;    // [N][2] entries, 16 bytes of the input zero point, [N] additive constants
    const int8_t* zfill;
    int32_t N, IC, IH, IW, OH, OW, pt, pl;
    int32_t row_tiles;  // per image
    int32_t ch_tiles;   // 32 CB channels each
    EpiArgs E;
};

constexpr int ROWS_RW = 7;    // output rows per producer wave
constexpr int ROWS_HWP = 32;  // halo positions per row (output rows of at most 30 pixels)

// LDS bytes of the row-tile kernel: halo image, two transfer buffers of
// two rows per producer wave, epilogue table.
constexpr size_t rows_lds(int cb)
{
    return size_t(4 / cb * ROWS_RW + 2) * ROWS_HWP * 128 + 2 * 4 * 2 * 4096 + size_t(cb) * 32 * 2 * 16;
}

template <int Q, int CB, int OB, bool RS, bool RC>
__global__ void __launch_bounds__(512, 1) conv_i8_rows_kernel(RowsArgs A)
{
    static_assert(Q == 4, "128 input channels");
    static_assert(CB == 2 || CB == 4, "64 or 128 channels per workgroup");
    static_assert(!RC || RS, "the range check belongs to the RESCALE");
    constexpr int RW = ROWS_RW;
    constexpr int RG = 4 / CB;  // producer waves along the rows
    constexpr int PB = 32 * Q;  // halo bytes per position
    constexpr int SL = 2 * Q;   // 16-byte chunks per position
    constexpr int HWP = ROWS_HWP;
    constexpr int HR = RG * RW + 2;
    constexpr int SLOTS = HR * HWP * SL;  // 16-byte halo slots
    constexpr int HBYTES = SLOTS * 16;
    constexpr int ROWB = HWP * PB;
    constexpr int XW = 2 * 4096;  // transfer bytes per producer wave and buffer (two rows)
    constexpr int XB = 4 * XW;    // transfer bytes per buffer
    static_assert(rows_lds(CB) == size_t(HBYTES + 2 * XB + 2 * 32 * CB * 16), "LDS layout");

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* const halo = smem;
    uint8_t* const xfer = smem + HBYTES;  // [2][4 waves][2 rows][4 chunks][64 lanes][16 B]
    v4i* const s_tab = reinterpret_cast<v4i*>(smem + HBYTES + 2 * XB);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pw = wave & 3;  // the producer wave (consumer wave pw + 4 serves it)
    const int cb = pw % CB, rg = pw / CB;
    const int l32 = lane & 31;
    const int h = lane >> 5;
    // Tile t of XCD x is workgroup x + 8 t (workgroups are dealt round-robin
    // to the XCDs), so that the channel tiles and neighbouring row tiles of
    // an image, which read the same input rows, meet in one L2.
    const int tile = (gridDim.x & 7) == 0 ? (blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int rt = tile / A.ch_tiles;
    const int ct = tile - rt * A.ch_tiles;
    const int img = rt / A.row_tiles;
    const int oy0 = (rt - img * A.row_tiles) * (RG * RW);
    const int n0 = ct * 32 * CB;
    const int nw = n0 + 32 * cb;  // the producer's first channel
    // Register slot q holds reduction chunk (q + rot) % Q: the sums do not
    // depend on the order, and workgroups that start at different chunks
    // spread their simultaneous weight requests over more L2 lines.
    const int rot = tile & (Q - 1);
    auto chunk = [&](int q) { return (q + rot) & (Q - 1); };

    // The halo is loaded in two parts: first the rows that each producer's
    // first phase reads (rows RW g .. RW g + 3 of row group g), then, behind
    // the weights, the other rows, which land in LDS while the first phase
    // computes. Slot o of a part (o = 512 i + tid) is chunk o % SL of
    // position (o / SL) % HWP of the part's row o / (SL HWP).
    constexpr int EROWS = 4 * RG;
    constexpr int ESLOTS = EROWS * HWP * SL;
    constexpr int LSLOTS = SLOTS - ESLOTS;
    static_assert(ESLOTS % 512 == 0, "whole early slots per thread");
    constexpr int NE = ESLOTS / 512;
    constexpr int NL = (LSLOTS + 511) / 512;
    // Halo row of the k-th row in load order: early rows RW g + 0..3, then
    // RW g + 4..6 of the groups before the last and the last group's rows
    // from RW (RG - 1) + 4 to the end.
    auto row_of = [](int k) {
        if (k < EROWS)
            return (k >> 2) * RW + (k & 3);
        k -= EROWS;
        const int g = k / 3;
        return g < RG - 1 ? g * RW + 4 + (k - 3 * g) : (RG - 1) * RW + 4 + (k - 3 * (RG - 1));
    };
    v4i hv_e[NE], hv_l[NL];
    int ho_e[NE], ho_l[NL];  // LDS byte offsets
    auto halo_load = [&](auto latec, v4i* hv, int* ho) {
        constexpr bool LATE = decltype(latec)::value;
        constexpr int NS = LATE ? LSLOTS : ESLOTS;
        constexpr int NN = LATE ? NL : NE;
        const int8_t* const xi = A.x + int64_t(img) * A.IH * A.IW * A.IC;
#pragma unroll
        for (int i = 0; i < NN; i++) {
            const int o = 512 * i + tid;
            if (512 * i + 64 * wave < NS) {
                const int hp = o / SL;
                const int hr = row_of(hp / HWP + (LATE ? EROWS : 0));
                const int pos = hp % HWP;
                const int c = (o % SL) ^ ((pos >> 1) % SL);
                const int iy = oy0 - A.pt + hr;
                const int ix = pos - A.pl;
                const bool ok = o < NS && unsigned(iy) < unsigned(A.IH) && unsigned(ix) < unsigned(A.IW);
                ho[i] = ((hr * HWP + pos) * SL + o % SL) * 16;
                hv[i] = *reinterpret_cast<const v4i*>(ok ? xi + (int64_t(iy) * A.IW + ix) * A.IC + 16 * c : A.zfill);
            }
        }
    };
    auto halo_store = [&](auto latec, const v4i* hv, const int* ho) {
        constexpr bool LATE = decltype(latec)::value;
        constexpr int NS = LATE ? LSLOTS : ESLOTS;
        constexpr int NN = LATE ? NL : NE;
#pragma unroll
        for (int i = 0; i < NN; i++)
            if (512 * i + 64 * wave < NS && 512 * i + tid < NS)
                *reinterpret_cast<v4i*>(halo + ho[i]) = hv[i];
    };
    using BF = std::integral_constant<bool, false>;
    using BT = std::integral_constant<bool, true>;

    using std::integral_constant;
    using I0 = integral_constant<int, 0>;
    using I1 = integral_constant<int, 1>;
    using I2 = integral_constant<int, 2>;
    using I4 = integral_constant<int, 4>;
    using I6 = integral_constant<int, 6>;
    static_assert(RW == 7, "phases of 2, 2, 2 and 1 rows");

    auto producer = [&]() {
        // Loads in the order of first use: the early halo rows, the
        // accumulators' constants, the weights in the order the first phase's
        // steps take them, the late halo rows.
        halo_load(BF{}, hv_e, ho_e);
        v16i init;  // the additive constants of this lane's channels nw + 16 h + i
        {
            const v4i* adds =
                reinterpret_cast<const v4i*>(reinterpret_cast<const int32_t*>(A.tab + 2 * A.N + 1) + nw + 16 * h);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const v4i v = adds[k];
                init[4 * k] = v.x;
                init[4 * k + 1] = v.y;
                init[4 * k + 2] = v.z;
                init[4 * k + 3] = v.w;
            }
        }
        v4i aw[Q][9];  // chunk q, tap t at ((block Q + chunk(q)) 9 + t) KB
        {
            const int8_t* const wsrc = A.wp + int64_t(nw >> 5) * (Q * 9 * 1024) + lane * 16;
#pragma unroll
            for (int q = 0; q < Q; q++)
#pragma unroll
                for (int kx = 0; kx < 3; kx++)
#pragma unroll
                    for (int ky = 0; ky < 3; ky++)
                        aw[q][3 * ky + kx] = *reinterpret_cast<const v4i*>(wsrc + (chunk(q) * 9 + 3 * ky + kx) * 1024);
        }
        halo_load(BT{}, hv_l, ho_l);
        halo_store(BF{}, hv_e, ho_e);
        __syncthreads();

        // Byte offsets of this lane's B fragments within a halo row: position
        // l32 + kx (clamped to the row; such lanes are past the output row),
        // chunk 2 q + h.
        int boff[3][Q];
#pragma unroll
        for (int kx = 0; kx < 3; kx++) {
            const int pos = l32 + kx < HWP ? l32 + kx : HWP - 1;
#pragma unroll
            for (int q = 0; q < Q; q++)
                boff[kx][q] = pos * PB + (((2 * chunk(q) + h) ^ ((pos >> 1) & (SL - 1))) << 4);
        }
        const uint8_t* const hb = halo + rg * RW * ROWB;

        // Rows R0 .. R0 + P - 1: step s = (q, kx) reads the next step's P + 2
        // B fragments and issues its 3 P MFMAs; the accumulators go to
        // transfer buffer BUF.
        auto phase = [&](auto r0c, auto pc, auto bufc) {
            constexpr int R0 = decltype(r0c)::value, P = decltype(pc)::value, BUF = decltype(bufc)::value;
            constexpr int S = 3 * Q, NM = 3 * P, ND = P + 2;
            v16i acc[P];
#pragma unroll
            for (int r = 0; r < P; r++)
                acc[r] = init;
            v4i bf[2][ND];
            auto ldb = [&](v4i(&bb)[ND], int st) {
                const int q = st / 3, kx = st - 3 * (st / 3);
#pragma unroll
                for (int j = 0; j < ND; j++)
                    bb[j] = *reinterpret_cast<const v4i*>(hb + (R0 + j) * ROWB + boff[kx][q]);
            };
            ldb(bf[0], 0);
#pragma unroll
            for (int st = 0; st < S; st++) {
                const int q = st / 3, kx = st - 3 * (st / 3);
                __builtin_amdgcn_sched_barrier(0);
                if (st + 1 < S)
                    ldb(bf[(st + 1) & 1], st + 1);
#pragma unroll
                for (int ky = 0; ky < 3; ky++)
#pragma unroll
                    for (int r = 0; r < P; r++)
                        acc[r] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aw[q][3 * ky + kx], bf[st & 1][r + ky], acc[r],
                                                                       0, 0, 0);
#pragma unroll
                for (int i = 0; i < NM; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                    if (i < ND && st + 1 < S)
                        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // Lane-contiguous 16-byte pieces: value group k of row r of lane l
            // at ((r 4 + k) 64 + l) 16.
            uint8_t* const xb = xfer + BUF * XB + pw * XW;
#pragma unroll
            for (int r = 0; r < P; r++)
#pragma unroll
                for (int k = 0; k < 4; k++)
                    *reinterpret_cast<v4i*>(xb + ((r * 4 + k) * 64 + lane) * 16) =
                        v4i{acc[r][4 * k], acc[r][4 * k + 1], acc[r][4 * k + 2], acc[r][4 * k + 3]};
        };
        phase(I0{}, I2{}, I0{});
        halo_store(BT{}, hv_l, ho_l);
        __syncthreads();
        phase(I2{}, I2{}, I1{});
        __syncthreads();
        phase(I4{}, I2{}, I0{});
        __syncthreads();
        phase(I6{}, I1{}, I1{});
        __syncthreads();
    };

    auto consumer = [&]() {
        halo_load(BF{}, hv_e, ho_e);
        const int ctid = tid - 256;
        v4i tv = v4i{0, 0, 0, 0};
        if (ctid < 2 * 32 * CB)
            tv = A.tab[2 * n0 + ctid];
        halo_store(BF{}, hv_e, ho_e);
        if (ctid < 2 * 32 * CB)
            s_tab[ctid] = tv;
        __syncthreads();
        // The consumers' share of the late rows, in LDS before the second
        // barrier.
        halo_load(BT{}, hv_l, ho_l);
        halo_store(BT{}, hv_l, ho_l);
        // Table entries of this lane's channels nw + 16 h + j.
        v4i t0[16], t1[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            t0[j] = s_tab[2 * (32 * cb + 16 * h + j)];
            if constexpr (RS)
                t1[j] = s_tab[2 * (32 * cb + 16 * h + j) + 1];
        }
        uint32_t bad_bits = 0;
        auto finish = [&](auto r0c, auto pc, auto bufc) {
            constexpr int R0 = decltype(r0c)::value, P = decltype(pc)::value, BUF = decltype(bufc)::value;
            const uint8_t* const xb = xfer + BUF * XB + pw * XW;
#pragma unroll
            for (int r = 0; r < P; r++) {
                v4i xv[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    xv[k] = *reinterpret_cast<const v4i*>(xb + ((r * 4 + k) * 64 + lane) * 16);
                uint32_t res[4 * OB];
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    int32_t v[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int j = 4 * g + i;
                        const int32_t x = xv[g][i];
                        if constexpr (RS) {
                            // apply_scale_32 with the per-sign rounding constant
                            // (the output zero point folded in), then the output
                            // range and CLAMP; with RC, its value-range REQUIRE.
                            if constexpr (RC)
                                bad_bits = __builtin_amdgcn_bitop3_b32(
                                    bad_bits, uint32_t(med3(x, t0[j].z, ~t0[j].z)), uint32_t(x), 0xf6);
                            const int64_t rp = __builtin_bit_cast(int64_t, v2i{t1[j].x, t1[j].y});
                            const int64_t rn = __builtin_bit_cast(int64_t, v2i{t1[j].z, t1[j].w});
                            const int32_t rr =
                                int32_t((int64_t(x) * int64_t(t0[j].y) + (x >= 0 ? rp : rn)) >> t0[j].w);
                            v[i] = med3(rr, A.E.clo, A.E.chi);
                        } else {
                            v[i] = x;
                        }
                    }
                    if constexpr (OB == 1) {
                        // Low bytes of v0..v3 (v_perm_b32: selector bytes 0-3
                        // pick the second operand, 4-7 the first, 0x0c zero).
                        const uint32_t p01 = __builtin_amdgcn_perm(uint32_t(v[1]), uint32_t(v[0]), 0x0c0c0400u);
                        const uint32_t p23 = __builtin_amdgcn_perm(uint32_t(v[3]), uint32_t(v[2]), 0x0c0c0400u);
                        res[g] = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
                    } else if constexpr (OB == 2) {
                        res[2 * g] = __builtin_amdgcn_perm(uint32_t(v[1]), uint32_t(v[0]), 0x05040100u);
                        res[2 * g + 1] = __builtin_amdgcn_perm(uint32_t(v[3]), uint32_t(v[2]), 0x05040100u);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            res[4 * g + i] = uint32_t(v[i]);
                    }
                }
                const int oy = oy0 + rg * RW + R0 + r;
                if (oy < A.OH && l32 < A.OW) {
                    const int64_t m = (int64_t(img) * A.OH + oy) * A.OW + l32;
                    uint8_t* const dst = A.E.out + (m * A.N + nw + 16 * h) * OB;
#pragma unroll
                    for (int wd = 0; wd < OB; wd++)
                        *reinterpret_cast<v4u*>(dst + 16 * wd) =
                            v4u{res[4 * wd], res[4 * wd + 1], res[4 * wd + 2], res[4 * wd + 3]};
                }
            }
        };
        __syncthreads();
        finish(I0{}, I2{}, I0{});
        __syncthreads();
        finish(I2{}, I2{}, I1{});
        __syncthreads();
        finish(I4{}, I2{}, I0{});
        __syncthreads();
        finish(I6{}, I1{}, I1{});
        if constexpr (RC) {
            if (bad_bits)
                atomicOr(A.E.err, DERR_SCALE_RANGE);
        }
    };
    // Both roles meet at the same five barriers.
    if (wave < 4)
        producer();
    else
        consumer();
}

// ---------------------------------------------------------------------------
// Streaming pointwise int8 convolution for short reductions (1x1, stride 1,
// K <= 64): a layer that moves K bytes in and N bytes out per pixel is
// memory-bound, and the tiled kernels' per-workgroup staging and barriers
// cost more than its MFMAs. Here the weights of a 32 TA-channel block live
// in VGPRs (A fragments in the halo kernel's row order, loaded once), the
// table in LDS, and every wave walks 32-pixel tiles on its own (no barriers
// after the prologue): per tile KS 16-byte loads per lane straight into B
// fragments (the next tile's are in flight while this one computes), TA x
// KS v_mfma_i32_32x32x32_i8, and the 32x32 epilogue. Reduction bytes past K
// load as zeros on both sides, so they add nothing to the dot products or to
// the weight zero point's per-pixel sums; the table's terms use the real K.
// K8: K % 16 == 8 (rows 8-byte aligned), every 16-byte piece loads as two
// 8-byte halves, each only where it lies inside the row.
// ---------------------------------------------------------------------------
struct PwsArgs {
    const int8_t* x;  // [M][K]
    const int8_t* w;  // [N][K]
    const v4i* tab;
    int32_t M, K, N;
    int32_t ntiles;  // 32-pixel tiles
    EpiArgs E;
};

template <int TA, int KS, int OB, bool RS, bool ZW, bool K8>
__global__ void __launch_bounds__(256, 2) conv_i8_pws_kernel(PwsArgs A)
{
    // 16 bytes of a row at byte k, zeros past K.
    auto ld_piece = [&](const int8_t* row, int k) -> v4i {
        if constexpr (!K8) {
            return k < A.K ? *reinterpret_cast<const v4i*>(row + k) : v4i{0, 0, 0, 0};
        } else {
            const v2i lo = k + 8 <= A.K ? *reinterpret_cast<const v2i*>(row + k) : v2i{0, 0};
            const v2i hi = k + 16 <= A.K ? *reinterpret_cast<const v2i*>(row + k + 8) : v2i{0, 0};
            return v4i{lo.x, lo.y, hi.x, hi.y};
        }
    };
    __shared__ v4i s_tab[2 * 32 * TA];
    __shared__ __attribute__((aligned(16))) int32_t s_add[32 * TA];  // additive constants
    __shared__ int32_t s_rowsum[4][32];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.y * 32 * TA;

    // Table entries of the block's channels (past N: channel N - 1).
    for (int i = tid; i < 2 * 32 * TA; i += 256) {
        const int c = n0 + (i >> 1);
        s_tab[i] = A.tab[2 * (c < A.N ? c : A.N - 1) + (i & 1)];
    }
    const int32_t* adds = reinterpret_cast<const int32_t*>(A.tab + 2 * A.N + 1);
    for (int i = tid; i < 32 * TA; i += 256)
        s_add[i] = adds[n0 + i < A.N ? n0 + i : A.N - 1];
    // A fragments: lane (row r = l32, k-half h) of channel tile a, step j
    // holds bytes 32 j + 16 h .. + 15 of channel n0 + 32 a + h32_row_channel(r).
    v4i wa[TA][KS];
#pragma unroll
    for (int a = 0; a < TA; a++) {
        const int c = n0 + 32 * a + h32_row_channel(l32);
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const int k = 32 * j + 16 * h;
            wa[a][j] = c < A.N ? ld_piece(A.w + int64_t(c) * A.K, k) : v4i{0, 0, 0, 0};
        }
    }
    __syncthreads();

    const int step = gridDim.x * 4;
    int t = blockIdx.x * 4 + wave;
    auto load_b = [&](int tile, v4i(&fb)[KS]) {
        const int p = 32 * tile + l32;
#pragma unroll
        for (int j = 0; j < KS; j++) {
            const int k = 32 * j + 16 * h;
            fb[j] = p < A.M ? ld_piece(A.x + int64_t(p) * A.K, k) : v4i{0, 0, 0, 0};
        }
    };
    v4i fb[KS], fn[KS];
    if (t < A.ntiles)
        load_b(t, fb);
    for (; t < A.ntiles; t += step) {
        if (t + step < A.ntiles)
            load_b(t + step, fn);
        if constexpr (ZW) {
            // Per-pixel sum of the input bytes: this lane's 16 bytes per
            // step, plus the other k-half's (lane l32 + 32).
            int32_t sx = 0;
#pragma unroll
            for (int j = 0; j < KS; j++) {
                sx = __builtin_amdgcn_sdot4(fb[j].x, 0x01010101, sx, false);
                sx = __builtin_amdgcn_sdot4(fb[j].y, 0x01010101, sx, false);
                sx = __builtin_amdgcn_sdot4(fb[j].z, 0x01010101, sx, false);
                sx = __builtin_amdgcn_sdot4(fb[j].w, 0x01010101, sx, false);
            }
            sx += __shfl_xor(sx, 32);
            if (h == 0)
                s_rowsum[wave][l32] = sx;
            __builtin_amdgcn_wave_barrier();
        }
        v16i acc[TA][1];
#pragma unroll
        for (int a = 0; a < TA; a++) {
            // Additive constants of this lane's result channels 32 a + 16 h + i.
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const v4i v = *reinterpret_cast<const v4i*>(s_add + 32 * a + 16 * h + 4 * q);
                acc[a][0][4 * q] = v.x;
                acc[a][0][4 * q + 1] = v.y;
                acc[a][0][4 * q + 2] = v.z;
                acc[a][0][4 * q + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < KS; j++)
                acc[a][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa[a][j], fb[j], acc[a][0], 0, 0, 0);
        }
        const int p0 = 32 * t;
        epilogue32<TA, 1, 1, OB, RS, ZW>(acc, s_tab, s_rowsum[wave], n0, 0, lane, A.E,
                                         [&](int p) { return p0 + p < A.M ? int64_t(p0 + p) : int64_t(-1); });
        if constexpr (ZW)
            __builtin_amdgcn_wave_barrier();  // the row sums are read before the next tile's
#pragma unroll
        for (int j = 0; j < KS; j++)
            fb[j] = fn[j];
    }
}

// Packed weights of the 32x32 halo kernel: 16-byte slot
// ((((nb passes + p) taps + t) TA + a) 64 + l) holds bytes 32 p + 16 (l / 32)
// .. + 15 of tap t of channel nb BC + 32 a + row_channel(l % 32) (zero past
// N), i.e. every pass of every channel block is the LDS image its loads fill.
__global__ void conv_i8_wpack_kernel(const int8_t* w, int32_t N, int32_t K, int32_t IC, int32_t taps, int32_t BC,
                                     int64_t slots, v4u* out)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= slots)
        return;
    const int TA = BC / 32, passes = IC / 32;
    int64_t r = i;
    const int l = int(r % 64);
    r /= 64;
    const int a = int(r % TA);
    r /= TA;
    const int t = int(r % taps);
    r /= taps;
    const int p = int(r % passes);
    const int nb = int(r / passes);
    const int c = nb * BC + 32 * a + h32_row_channel(l % 32);
    v4u v = v4u{0, 0, 0, 0};
    if (c < N)
        v = *reinterpret_cast<const v4u*>(w + int64_t(c) * K + t * IC + 32 * p + 16 * (l / 32));
    out[i] = v;
}

// ---------------------------------------------------------------------------
// Materialised im2col for the convolutions the tiled kernels do not take
// directly (input channels that are not a multiple of the stage width, e.g.
// a 3-channel stem): X~[m][k], k = (ky KW + kx) IC + ic < K, holds the input
// byte at the tap (the input zero point outside the input, which the
// zero-point fold turns into the reference's skipped tap), and K <= k < Kp
// holds 0 (a zero weight column multiplies it). The pointwise kernel then
// runs over X~ with the weights padded to [OC][Kp]. One thread per 16-byte
// chunk (blockIdx.y) of one row (pixel); the tap of each byte is uniform.
// ---------------------------------------------------------------------------
struct Im2colArgs {
    const int8_t* x;
    int8_t* out;
    int32_t M, K, Kp, IC;
    int32_t ih, iw, kw, ohow, ow, pt, pl, sy, sx, dy, dx;
    FastDiv div_ohow, div_ow;
    int32_t zp_x;
};

__global__ void __launch_bounds__(256) conv_i8_im2col_kernel(Im2colArgs A)
{
    const int m = blockIdx.x * 256 + threadIdx.x;
    if (m >= A.M)
        return;
    const int k0 = blockIdx.y * 16;
    const int b = fdiv(m, A.div_ohow);
    const int rem = m - b * A.ohow;
    const int oy = fdiv(rem, A.div_ow);
    const int ox = rem - oy * A.ow;
    const int iy0 = oy * A.sy - A.pt, ix0 = ox * A.sx - A.pl;
    const int8_t* xb = A.x + int64_t(b) * A.ih * A.iw * A.IC;
    uint32_t wv[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int k = k0 + j;
        uint32_t v = 0;
        if (k < A.K) {
            const int t = k / A.IC, ic = k - t * A.IC;
            const int ky = t / A.kw, kx = t - ky * A.kw;
            const int iy = iy0 + ky * A.dy, ix = ix0 + kx * A.dx;
            const bool ok = unsigned(iy) < unsigned(A.ih) && unsigned(ix) < unsigned(A.iw);
            v = ok ? uint8_t(xb[(int64_t(iy) * A.iw + ix) * A.IC + ic]) : uint8_t(A.zp_x);
        }
        wv[j >> 2] |= v << (8 * (j & 3));
    }
    *reinterpret_cast<v4u*>(A.out + int64_t(m) * A.Kp + k0) = v4u{wv[0], wv[1], wv[2], wv[3]};
}

// The same with the taps of the first IM2COL_TAB columns tabulated on the
// host (a uniform kernel argument per column: its offset from the pixel's
// origin, or -1 past K, and its row and column displacement), so a column
// costs one load and a bounds test. DW4: IC % 4 == 0, four columns of one
// tap per 32-bit load.
constexpr int IM2COL_TAB = 128;
struct Im2colTab {
    int32_t off[IM2COL_TAB];
    int16_t dy[IM2COL_TAB], dx[IM2COL_TAB];
};

template <bool DW4>
__global__ void __launch_bounds__(256) conv_i8_im2col_tab_kernel(Im2colArgs A, Im2colTab T)
{
    const int m = blockIdx.x * 256 + threadIdx.x;
    if (m >= A.M)
        return;
    const int k0 = blockIdx.y * 16;
    const int b = fdiv(m, A.div_ohow);
    const int rem = m - b * A.ohow;
    const int oy = fdiv(rem, A.div_ow);
    const int ox = rem - oy * A.ow;
    const int iy0 = oy * A.sy - A.pt, ix0 = ox * A.sx - A.pl;
    const int8_t* xp = A.x + int64_t(b) * A.ih * A.iw * A.IC + (int64_t(iy0) * A.iw + ix0) * A.IC;
    const uint32_t zf = uint32_t(uint8_t(A.zp_x)) * 0x01010101u;
    uint32_t wv[4] = {0, 0, 0, 0};
    if constexpr (DW4) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = k0 + 4 * q;
            const int o = T.off[k];
            if (o >= 0) {
                const int iy = iy0 + T.dy[k], ix = ix0 + T.dx[k];
                const bool ok = unsigned(iy) < unsigned(A.ih) && unsigned(ix) < unsigned(A.iw);
                wv[q] = ok ? *reinterpret_cast<const uint32_t*>(xp + o) : zf;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int k = k0 + j;
            const int o = T.off[k];
            if (o >= 0) {
                const int iy = iy0 + T.dy[k], ix = ix0 + T.dx[k];
                const bool ok = unsigned(iy) < unsigned(A.ih) && unsigned(ix) < unsigned(A.iw);
                const uint32_t v = ok ? uint8_t(xp[o]) : uint8_t(A.zp_x);
                wv[j >> 2] |= v << (8 * (j & 3));
            }
        }
    }
    *reinterpret_cast<v4u*>(A.out + int64_t(m) * A.Kp + k0) = v4u{wv[0], wv[1], wv[2], wv[3]};
}

// Rows of K bytes copied into rows of Kp >= K bytes, zero-filled.
__global__ void conv_i8_rowpad_kernel(const int8_t* w, int32_t rows, int32_t K, int32_t Kp, int8_t* out)
{
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(rows) * Kp)
        return;
    const int64_t r = i / Kp;
    const int k = int(i - r * Kp);
    out[i] = k < K ? w[r * K + k] : int8_t(0);
}

// B [batch][C][W] -> [batch][W][C] (the MATMUL right operand as OHWI-style
// rows of C bytes): a workgroup moves TT 64 x 64 byte tiles along W through
// LDS, all of their loads issued before the first LDS write. C % 16 == 0;
// VEC: W % 16 == 0, so the rows of B load as 16-byte vectors.
constexpr int TR_TT = 4;

template <bool VEC>
__global__ void __launch_bounds__(256) transpose_b_kernel(const int8_t* b, int32_t C, int32_t W, int8_t* out)
{
    __shared__ uint8_t t[TR_TT][64][64 + 4];
    const int z = blockIdx.z;
    const int c0 = blockIdx.y * 64, w00 = blockIdx.x * (64 * TR_TT);
    const int8_t* src = b + int64_t(z) * C * W;
    int8_t* dst = out + int64_t(z) * C * W;
    const int r = threadIdx.x >> 2, q = threadIdx.x & 3;
    // load: row c0 + r, columns w0 + 16 q .. + 15 of each tile
    uint32_t v[TR_TT][4];
    const int c = c0 + r;
#pragma unroll
    for (int tt = 0; tt < TR_TT; tt++) {
        const int w = w00 + 64 * tt + 16 * q;
#pragma unroll
        for (int j = 0; j < 4; j++)
            v[tt][j] = 0;
        if (c < C) {
            if (VEC) {
                if (w < W) {
                    const v4u x = *reinterpret_cast<const v4u*>(src + int64_t(c) * W + w);
                    v[tt][0] = x.x;
                    v[tt][1] = x.y;
                    v[tt][2] = x.z;
                    v[tt][3] = x.w;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 16; j++)
                    if (w + j < W)
                        v[tt][j >> 2] |= uint32_t(uint8_t(src[int64_t(c) * W + w + j])) << (8 * (j & 3));
            }
        }
    }
#pragma unroll
    for (int tt = 0; tt < TR_TT; tt++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            *reinterpret_cast<uint32_t*>(&t[tt][r][16 * q + 4 * j]) = v[tt][j];
    __syncthreads();
    // store: output row w0 + r, columns c0 + 16 q .. + 15 of each tile
    const int cc = c0 + 16 * q;
#pragma unroll
    for (int tt = 0; tt < TR_TT; tt++) {
        const int w = w00 + 64 * tt + r;
        if (w >= W || cc >= C)
            continue;
        uint32_t o[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < 16; j++)
            o[j >> 2] |= uint32_t(t[tt][16 * q + j][r]) << (8 * (j & 3));
        *reinterpret_cast<v4u*>(dst + int64_t(w) * C + cc) = v4u{o[0], o[1], o[2], o[3]};
    }
}

// ---------------------------------------------------------------------------
// DEPTHWISE_CONV2D (depth multiplier 1) on MFMA
// ---------------------------------------------------------------------------
// For 16 channels c0..c0+15 and 16 output pixels, the depthwise sum
// out[c][p] = sum_t w[t][c] x~[p, t][c] is a 16 x 16 x (16 channels x 4 taps)
// MFMA whose A operand is block-diagonal: lane (row c, k-chunk = tap t) holds
// w[t][c] in byte c of its 16 bytes and zero elsewhere, and the B operand is
// the plain 16-byte NHWC load of the channel group at (pixel, tap). Three
// v_mfma_i32_16x16x64_i8 cover up to 12 taps (3x3 plus 3 zero taps); VALU
// work is left to the epilogue alone. Zero points fold as in CONV2D with
// K = taps: the per-channel terms come from the table, the per-(pixel,
// channel) term zw sum_t x~ from a second MFMA against block-diagonal ones.
//
// A workgroup covers 64 consecutive output pixels (flattened n, oy, ox) and
// 4 consecutive channel groups, one per wave, so that its waves read the same
// input lines (L1 reuse) and each wave issues all its loads at once.
struct DwArgs {
    const int8_t* x;
    const int8_t* w;
    const v4i* tab;
    int32_t P, C, IH, IW, OH, OW, KW, T, sy, sx, dy, dx, pt, pl;
    FastDiv div_ohow, div_ow;
    int32_t zp_x;
    EpiArgs E;
};

template <int G, int OB, bool RS, bool ZW>
__global__ void __launch_bounds__(256, 4) conv_i8_dw_kernel(DwArgs A)
{
    constexpr int TN = 4;  // 16-pixel tiles per wave
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j16 = lane & 15;
    const int grp = lane >> 4;
    // Work item of the wave: (64-pixel tile, 16-channel group), channel
    // groups fastest, so every wave has work whatever the channel count and
    // the waves of a workgroup read neighbouring channels of the same pixels.
    const int groups = A.C >> 4;
    const int item = blockIdx.x * 4 + wave;
    const int ptile = item / groups;
    const int cg = item - ptile * groups;
    const int p0 = ptile * (16 * TN);
    if (p0 >= A.P)
        return;

    // Input offsets of this lane's pixel in each tile (without the tap) and
    // the tap of each of its k-chunks: tap 4 g + grp of group g.
    int32_t iy0[TN], ix0[TN], pbase[TN];
    bool pok[TN];
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int p = p0 + 16 * tn + j16;
        pok[tn] = p < A.P;
        const int pp = pok[tn] ? p : 0;
        const int b = fdiv(pp, A.div_ohow);
        const int rem = pp - b * (A.OH * A.OW);
        const int oy = fdiv(rem, A.div_ow);
        const int ox = rem - oy * A.OW;
        iy0[tn] = oy * A.sy - A.pt;
        ix0[tn] = ox * A.sx - A.pl;
        pbase[tn] = b * A.IH * A.IW;
    }
    int32_t tdy[G], tdx[G];
    bool tok[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int t = 4 * g + grp;
        tok[g] = t < A.T;
        const int ky = t / A.KW;
        tdy[g] = ky * A.dy;
        tdx[g] = (t - ky * A.KW) * A.dx;
    }

    {
        const int c0 = cg * 16;
        // Block-diagonal A fragments: byte j16 of 16 is w[t][c0 + j16].
        v4i wa[G], wo[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            const int t = 4 * g + grp;
            const uint32_t wv = tok[g] ? uint32_t(uint8_t(A.w[t * A.C + c0 + j16])) : 0u;
            const int sh = 8 * (j16 & 3);
            const int wd = j16 >> 2;
            wa[g] = v4i{wd == 0 ? int(wv << sh) : 0, wd == 1 ? int(wv << sh) : 0, wd == 2 ? int(wv << sh) : 0,
                        wd == 3 ? int(wv << sh) : 0};
            if constexpr (ZW) {
                const uint32_t one = tok[g] ? 1u : 0u;
                wo[g] = v4i{wd == 0 ? int(one << sh) : 0, wd == 1 ? int(one << sh) : 0,
                            wd == 2 ? int(one << sh) : 0, wd == 3 ? int(one << sh) : 0};
            }
        }
        // Table of the 4 output channels this lane holds: c0 + 4 grp + i.
        v4i t0[4], t1[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            t0[i] = A.tab[2 * (c0 + 4 * grp + i)];
            if constexpr (RS)
                t1[i] = A.tab[2 * (c0 + 4 * grp + i) + 1];
        }
        int32_t hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            hi[i] = ~t0[i].z;
        uint32_t bad_bits = 0;
        // Every tap of the wave's four tiles is loaded before the first
        // MFMA: padding taps read the table's 16 bytes of input zero point,
        // so no load is conditional (a select after the load lets the
        // compiler put each load behind a branch and wait for it alone).
        const int8_t* const zfill = reinterpret_cast<const int8_t*>(A.tab + 2 * A.C);
        v4u xin[TN][G];
#pragma unroll
        for (int tn = 0; tn < TN; tn++)
#pragma unroll
            for (int g = 0; g < G; g++) {
                const int iy = iy0[tn] + tdy[g];
                const int ix = ix0[tn] + tdx[g];
                const bool ok = tok[g] && unsigned(iy) < unsigned(A.IH) && unsigned(ix) < unsigned(A.IW);
                xin[tn][g] = ld16(ok ? A.x + (pbase[tn] + iy * A.IW + ix) * A.C + c0 : zfill);
            }
        // RC: some shift is below 32, so the value-range REQUIRE is checked.
        auto tiles = [&](auto rc) {
            constexpr bool RC = decltype(rc)::value;
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            v4i acc = v4i{0, 0, 0, 0}, acc1 = v4i{0, 0, 0, 0};
#pragma unroll
            for (int g = 0; g < G; g++) {
                const v4i bx = __builtin_bit_cast(v4i, xin[tn][g]);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[g], bx, acc, 0, 0, 0);
                if constexpr (ZW)
                    acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wo[g], bx, acc1, 0, 0, 0);
            }
            if (!pok[tn])
                continue;
            int32_t v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t xu = uint32_t(acc[i]) + uint32_t(t0[i].x);
                if constexpr (ZW)
                    xu += uint32_t(-A.E.zp_w) * uint32_t(acc1[i]);
                const int32_t xv = int32_t(xu);
                if constexpr (RS) {
                    if constexpr (RC)
                        bad_bits = __builtin_amdgcn_bitop3_b32(bad_bits, uint32_t(med3(xv, t0[i].z, hi[i])),
                                                               uint32_t(xv), 0xf6);  // bad | (med3 ^ x)
                    const int64_t rp = __builtin_bit_cast(int64_t, v2i{t1[i].x, t1[i].y});
                    const int64_t rn = __builtin_bit_cast(int64_t, v2i{t1[i].z, t1[i].w});
                    const int32_t r = int32_t((int64_t(xv) * int64_t(t0[i].y) + (xv >= 0 ? rp : rn)) >> t0[i].w);
                    v[i] = med3(r, A.E.clo, A.E.chi);
                } else {
                    v[i] = xv;
                }
            }
            uint8_t* dst = A.E.out + (int64_t(p0 + 16 * tn + j16) * A.C + c0 + 4 * grp) * OB;
            if constexpr (OB == 1)
                *reinterpret_cast<uint32_t*>(dst) = pack4_u8(v[0], v[1], v[2], v[3]);
            else if constexpr (OB == 2)
                *reinterpret_cast<v2u*>(dst) = v2u{(uint32_t(v[0]) & 0xFFFF) | (uint32_t(v[1]) << 16),
                                                   (uint32_t(v[2]) & 0xFFFF) | (uint32_t(v[3]) << 16)};
            else
                *reinterpret_cast<v4i*>(dst) = v4i{v[0], v[1], v[2], v[3]};
            if constexpr (RS && RC)
                asm volatile("" : "+v"(bad_bits));
        }
        };
        if (!RS || A.E.range)
            tiles(std::true_type{});
        else
            tiles(std::false_type{});
        if (bad_bits)
            atomicOr(A.E.err, DERR_SCALE_RANGE);
    }
}

// One wave per output channel:
//   tab[2c]   = {bias + K zx zw - zx sum_k w[c][k] (mod 2^32), multiplier,
//                -2^min(shift - 1, 31), shift}
//               with the third word INT32_MIN instead when the channel's
//               values cannot leave [-2^(shift-1), 2^(shift-1)):
//               |bias| + max|x - zx| sum_k |w[c][k] - zw| < 2^(shift-1)
//   tab[2c+1] = {rounding constant for values >= 0 (int64, lo/hi),
//                rounding constant for values < 0 (int64, lo/hi)},
//                both plus out_zp 2^shift
// then, after the N channels, 16 bytes of the input zero point and the N
// additive constants (tab[2c].x) as a dense array. The
// rounding constants are apply_scale_32's 2^(s-1), plus or minus 2^30 under
// double rounding for shifts above 31 (src/ops/quant.rs:26-29).
__global__ void conv_i8_table_kernel(const int8_t* w, int32_t N, int32_t K, int32_t cstride, int32_t kstride,
                                     const int32_t* bias, int32_t bias_len, int32_t zx, int32_t zw,
                                     const int32_t* mult, const int32_t* shift, int32_t per_channel, int32_t dbl,
                                     int32_t out_zp, v4i* tab, int64_t wbatch, int32_t tbatch)
{
    const int c = blockIdx.x;
    const int lane = threadIdx.x;
    w += blockIdx.y * wbatch;
    tab += blockIdx.y * tbatch;
    if (c == 0 && lane == 0) {
        const int32_t zf = int32_t(uint32_t(uint8_t(zx)) * 0x01010101u);
        tab[2 * N] = v4i{zf, zf, zf, zf};
    }
    // s: sum_k w; sa: sum_k |w - zw| (bytes biased by 128 to unsigned, which
    // keeps differences, then v_sad_u8), the latter only with a RESCALE.
    int32_t s = 0;
    uint32_t sa = 0;
    if (w && (zx != 0 || mult)) {
        const int8_t* wr = w + int64_t(c) * cstride;
        const uint32_t zwb = (uint32_t(uint8_t(zw)) * 0x01010101u) ^ 0x80808080u;
        if (kstride == 1 && K % 16 == 0 && reinterpret_cast<uintptr_t>(wr) % 16 == 0) {
            // Contiguous rows: 16 bytes per lane per step, summed with dot4.
            for (int k = 16 * lane; k < K; k += 16 * 64) {
                const v4u v = *reinterpret_cast<const v4u*>(wr + k);
                s = __builtin_amdgcn_sdot4(int(v.x), 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4(int(v.y), 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4(int(v.z), 0x01010101, s, false);
                s = __builtin_amdgcn_sdot4(int(v.w), 0x01010101, s, false);
                sa = __builtin_amdgcn_sad_u8(v.x ^ 0x80808080u, zwb, sa);
                sa = __builtin_amdgcn_sad_u8(v.y ^ 0x80808080u, zwb, sa);
                sa = __builtin_amdgcn_sad_u8(v.z ^ 0x80808080u, zwb, sa);
                sa = __builtin_amdgcn_sad_u8(v.w ^ 0x80808080u, zwb, sa);
            }
        } else {
            for (int k = lane; k < K; k += 64) {
                const int32_t v = wr[int64_t(k) * kstride];
                s += v;
                sa += uint32_t(v > zw ? v - zw : zw - v);
            }
        }
    }
    // Lane sums stay below 2^32 for K < 2^24 / 255 per lane.
    uint64_t sa64 = sa;
    for (int off = 32; off > 0; off >>= 1) {
        s += __shfl_xor(s, off);
        sa64 += __shfl_xor(sa64, off);
    }
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
    // The output zero point rides in the rounding constants: (P + R) >> s
    // + zp == (P + R + zp 2^s) >> s, and the host admits only zero points
    // with |zp| 2^s <= 2^60, so P + R + zp 2^s stays inside int64.
    const int64_t zps = int64_t(out_zp) * (int64_t(1) << sh);
    const int64_t rp = half + d + zps, rn = half - d + zps;
    // Range bound of apply_scale_32's REQUIRE: values in [lo, ~lo] with
    // lo = -2^min(s - 1, 31).
    int32_t lo = sh - 1 < 31 ? -(int32_t(1) << (sh - 1)) : INT32_MIN;
    if (w && mult && lo != INT32_MIN) {
        const int64_t b = bias ? int64_t(bias[bias_len == 1 ? 0 : c]) : 0;
        const int64_t xmax = std::max<int64_t>(128 + int64_t(zx), 127 - int64_t(zx));
        const uint64_t bound = uint64_t(b < 0 ? -b : b) + sa64 * uint64_t(xmax);
        if (K < (1 << 24) && bound < (uint64_t(1) << (sh - 1)))  // K bound: no lane sum overflow
            lo = INT32_MIN;
    }
    tab[2 * c] = v4i{int32_t(add), m, lo, sh};
    reinterpret_cast<int32_t*>(tab + 2 * N + 1)[c] = int32_t(add);
    tab[2 * c + 1] = v4i{int32_t(uint32_t(uint64_t(rp))), int32_t(uint64_t(rp) >> 32),
                         int32_t(uint32_t(uint64_t(rn))), int32_t(uint64_t(rn) >> 32)};
}

template <int TA, int KS, bool ZW, bool K8 = false>
void launch_pws(const PwsArgs& a, hipStream_t s)
{
    const unsigned wgs = unsigned(std::min<int64_t>((a.ntiles + 3) / 4, int64_t(2) * cu_count()));
    hipLaunchKernelGGL((conv_i8_pws_kernel<TA, KS, 1, true, ZW, K8>),
                       dim3(wgs, unsigned((a.N + 32 * TA - 1) / (32 * TA))), dim3(256), 0, s, a);
}

// Channel tiles per block: the most of 4, 3, 2, 1 that divide N / 32 (with
// K % 16 == 8, up to three and the last block partial).
template <int KS, bool ZW>
void launch_pws_ta(const PwsArgs& a, hipStream_t s)
{
    const int t = a.N / 32;
    if (a.K % 16 == 8) {
        // Up to three 32-channel tiles per block (the last block partial).
        const int tiles = (a.N + 31) / 32;
        if (tiles >= 3)
            launch_pws<3, KS, ZW, true>(a, s);
        else if (tiles == 2)
            launch_pws<2, KS, ZW, true>(a, s);
        else
            launch_pws<1, KS, ZW, true>(a, s);
        return;
    }
    if (t % 4 == 0)
        launch_pws<4, KS, ZW>(a, s);
    else if (t % 3 == 0)
        launch_pws<3, KS, ZW>(a, s);
    else if (t % 2 == 0)
        launch_pws<2, KS, ZW>(a, s);
    else
        launch_pws<1, KS, ZW>(a, s);
}

// ---------------------------------------------------------------------------
// Stem convolution: 3x3 taps over 3 input channels (K = 27 bytes per output
// pixel), the MobileNet-style first layer, without a materialised im2col. A
// workgroup owns R output rows of one image and stages the input rows they
// read in LDS as one 32-bit word per pixel (3 channel bytes, a zero byte), the
// padding columns and rows holding the input zero point; a global row of 4
// pixels is 12 bytes, loaded as three words and spread with byte permutes.
// The 32-byte reduction row of an output pixel in (ky, kx, c) order then is
// six aligned LDS words -- rows ky = h, h + 1 of the lane's k-half h -- put
// together with four v_perm_b32 (bytes 27-31 zero, as are the padded weights'
// there). Weights of 32 channels stay in VGPRs and the epilogue is the
// streaming pointwise kernel's.
// ---------------------------------------------------------------------------
struct StemArgs {
    const int8_t* x;  // NHWC [n][IH][IW][3]
    const int8_t* w;  // [N][32]: the 27 weights of a channel, then zeros
    const v4i* tab;
    int32_t N, IH, IW, OH, OW, sy, sx, pt, pl;
    int32_t R, bands, units;  // output rows per workgroup, bands per image, images x bands
    int32_t HR, WP;           // staged input rows and padded row width (pixels)
    uint32_t zfw;             // a padding pixel: three zero-point bytes
    FastDiv div_ow, div_bands, div_g;
    EpiArgs E;
};

template <bool ZW>
__global__ void __launch_bounds__(256, 2) conv_i8_stem_kernel(StemArgs A)
{
    extern __shared__ uint32_t s_px[];  // [HR][WP]
    __shared__ v4i s_tab[2 * 32];
    __shared__ __attribute__((aligned(16))) int32_t s_add[32];
    __shared__ int32_t s_rowsum[4][32];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int n0 = blockIdx.y * 32;

    for (int i = tid; i < 2 * 32; i += 256) {
        const int c = n0 + (i >> 1);
        s_tab[i] = A.tab[2 * (c < A.N ? c : A.N - 1) + (i & 1)];
    }
    const int32_t* adds = reinterpret_cast<const int32_t*>(A.tab + 2 * A.N + 1);
    for (int i = tid; i < 32; i += 256)
        s_add[i] = adds[n0 + i < A.N ? n0 + i : A.N - 1];
    // A fragment: lane (row l32, k-half h) holds bytes 16 h .. + 15 of
    // channel n0 + h32_row_channel(l32).
    v4i wa;
    {
        const int c = n0 + h32_row_channel(l32);
        wa = c < A.N ? *reinterpret_cast<const v4i*>(A.w + int64_t(c) * 32 + 16 * h) : v4i{0, 0, 0, 0};
    }
    const int groups = A.IW >> 2;  // 4-pixel groups of an input row

    for (int u = blockIdx.x; u < A.units; u += gridDim.x) {
        const int img = fdiv(u, A.div_bands);
        const int oy0 = (u - img * A.bands) * A.R;
        const int rows = A.OH - oy0 < A.R ? A.OH - oy0 : A.R;
        const int iy0 = oy0 * A.sy - A.pt;
        __syncthreads();  // the previous band's reads are done
        // Interior pixels, 4 at a time.
        for (int i = tid; i < A.HR * groups; i += 256) {
            const int hr = fdiv(i, A.div_g);
            const int g = i - hr * groups;
            const int iy = iy0 + hr;
            uint32_t* dst = s_px + hr * A.WP + A.pl + 4 * g;
            if (unsigned(iy) < unsigned(A.IH)) {
                const uint32_t* src =
                    reinterpret_cast<const uint32_t*>(A.x + ((int64_t(img) * A.IH + iy) * A.IW + 4 * g) * 3);
                const uint32_t d0 = src[0], d1 = src[1], d2 = src[2];
                dst[0] = d0 & 0xffffffu;
                dst[1] = __builtin_amdgcn_perm(d1, d0, 0x0c050403u);
                dst[2] = __builtin_amdgcn_perm(d2, d1, 0x0c040302u);
                dst[3] = d2 >> 8;
            } else {
                dst[0] = dst[1] = dst[2] = dst[3] = A.zfw;
            }
        }
        // Padding columns left and right of the image.
        const int pr = A.WP - A.pl - A.IW;
        for (int i = tid; i < A.HR * (A.pl + pr); i += 256) {
            const int hr = i / (A.pl + pr);
            const int c = i - hr * (A.pl + pr);
            s_px[hr * A.WP + (c < A.pl ? c : A.IW + c)] = A.zfw;
        }
        __syncthreads();

        const int npx = rows * A.OW;
        const int ntl = (npx + 31) >> 5;
        const int64_t m0 = (int64_t(img) * A.OH + oy0) * A.OW;
        for (int t = wave; t < ntl; t += 4) {
            const int p = 32 * t + l32;
            const int pc = p < npx ? p : 0;
            const int r = fdiv(pc, A.div_ow);
            const int ox = pc - r * A.OW;
            // Words of taps (h, 0..2) and (h + 1, 0..2).
            const uint32_t* q = s_px + (r * A.sy + h) * A.WP + ox * A.sx;
            const uint32_t a0 = q[0], a1 = q[1], a2 = q[2];
            const uint32_t b0 = q[A.WP], b1 = q[A.WP + 1], b2 = q[A.WP + 2];
            v4i fb;
            if (h == 0) {
                fb = v4i{int(__builtin_amdgcn_perm(a1, a0, 0x04020100u)), int(__builtin_amdgcn_perm(a2, a1, 0x05040201u)),
                         int(__builtin_amdgcn_perm(b0, a2, 0x06050402u)), int(__builtin_amdgcn_perm(b2, b1, 0x04020100u))};
            } else {
                fb = v4i{int(__builtin_amdgcn_perm(b0, a2, 0x05040201u)), int(__builtin_amdgcn_perm(b1, b0, 0x06050402u)),
                         int(b2), 0};
            }
            if constexpr (ZW) {
                int32_t sxs = 0;
                sxs = __builtin_amdgcn_sdot4(fb.x, 0x01010101, sxs, false);
                sxs = __builtin_amdgcn_sdot4(fb.y, 0x01010101, sxs, false);
                sxs = __builtin_amdgcn_sdot4(fb.z, 0x01010101, sxs, false);
                sxs = __builtin_amdgcn_sdot4(fb.w, 0x01010101, sxs, false);
                sxs += __shfl_xor(sxs, 32);
                if (h == 0)
                    s_rowsum[wave][l32] = sxs;
                __builtin_amdgcn_wave_barrier();
            }
            v16i acc[1][1];
#pragma unroll
            for (int qd = 0; qd < 4; qd++) {
                const v4i v = *reinterpret_cast<const v4i*>(s_add + 16 * h + 4 * qd);
                acc[0][0][4 * qd] = v.x;
                acc[0][0][4 * qd + 1] = v.y;
                acc[0][0][4 * qd + 2] = v.z;
                acc[0][0][4 * qd + 3] = v.w;
            }
            acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wa, fb, acc[0][0], 0, 0, 0);
            const int p0 = 32 * t;
            epilogue32<1, 1, 1, 1, true, ZW>(acc, s_tab, s_rowsum[wave], n0, 0, lane, A.E,
                                            [&](int pp) { return p0 + pp < npx ? m0 + p0 + pp : int64_t(-1); });
            if constexpr (ZW)
                __builtin_amdgcn_wave_barrier();  // the row sums are read before the next tile's
        }
    }
}

// The streaming pointwise kernel takes 1x1 stride-1 convolutions with
// K = ic a multiple of 16 up to 64, N a multiple of 32 (its epilogue works on
// whole 32-channel tiles: with N = 16, 24 or 144 the padded channels made it
// no faster than the tiled kernel), many pixels (its persistent waves need
// tiles to walk) and the fused RESCALE to int8. With K % 16 == 8 (24, 40,
// 56 channels: otherwise an im2col pad copy and the tiled kernel) it also
// takes N a multiple of 16, in one-tile channel blocks.
bool pws_applies(const ConvI8Desc& d, bool pw, int ob, const RescaleDev* rs)
{
    const int64_t m = int64_t(d.n) * d.oh * d.ow;
    const uintptr_t al = reinterpret_cast<uintptr_t>(d.x) | reinterpret_cast<uintptr_t>(d.w);
    const bool k16 = d.ic % 16 == 0 && d.oc % 32 == 0 && al % 16 == 0;
    const bool k8 = d.ic % 16 == 8 && d.oc % 16 == 0 && al % 8 == 0;
    return pw && d.batch == 1 && rs && ob == 1 && (k16 || k8) && d.ic <= 64 && m >= 4096 &&
           m * d.ic < (int64_t(1) << 31);
}

template <int BC, int BP, int WC, int WP, int KC, bool PW, int OB, bool RS, bool ZW, bool RES = false>
void launch(const ConvI8Args& a, hipStream_t s)
{
    auto kfn = conv_i8_kernel<BC, BP, WC, WP, KC, PW, OB, RS, ZW, RES>;
    constexpr size_t lds =
        size_t(2) * (BC + BP) * KC + size_t(32) * BC + (RES ? size_t(4) * CONV_I8_RES_WORDS * BC : 0);
    static_assert(lds >= 4 * BP, "rowsum scratch");
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      int(lds)),
                  "conv_i8 LDS size");
        return true;
    }();
    (void)attr;
    dim3 grid((a.M + BP - 1) / BP, (a.N + BC - 1) / BC, PW ? a.batch : 1);
    hipLaunchKernelGGL(kfn, grid, dim3(256), lds, s, a);
}

template <int BC, int BP, int WC, int WP, int KC, bool PW>
void launch_epi(const ConvI8Args& a, int ob, bool rs, bool zw, hipStream_t s, bool res = false)
{
    // Tiles of at most eight accumulator fragments per wave take the residual
    // stage: its per-channel constants and skip bytes would make the
    // sixteen-fragment tiles (128 x 128, 64 x 256) spill registers.
    constexpr bool RES_OK = PW && (BC / WC / 16) * (BP / WP / 16) <= 8;
    if constexpr (RES_OK) {
        if (res) {
            // The quantised residual follows an int8 RESCALE (host-checked).
            if (zw)
                launch<BC, BP, WC, WP, KC, PW, 1, true, true, true>(a, s);
            else
                launch<BC, BP, WC, WP, KC, PW, 1, true, false, true>(a, s);
            return;
        }
    }
    if (res)
        throw std::logic_error("conv_i8: residual stage on a tile without it");
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

// Channel tile with the least padded channel work (the 128-channel tile
// skips a 64-channel half past N), the wider tile on a tie: the epilogue's
// per-output work dominates layers with few reduction steps. Pointwise
// layers weigh the input's re-reads per channel block instead.
template <int KC, bool PW>
void launch_tile(const ConvI8Args& a, int ob, bool rs, bool zw, hipStream_t s, bool res = false)
{
    const int64_t n = a.N;
    const int64_t w128 = (n + 63) / 64 * 64, w64 = (n + 63) / 64 * 64, w32 = (n + 31) / 32 * 32,
                  w16 = (n + 15) / 16 * 16;
    if (PW && a.M >= 32768) {
        // Pointwise layers over many pixels are mostly memory-bound (a 1x1
        // convolution reads K bytes per pixel and channel block): cost =
        // re-reads of the input per channel block, weighted 64 to 1 against
        // the padded channel work. The widest tile wins ties. (Over few
        // pixels, narrow tiles give the workgroups that fill the chip.)
        const int64_t cost[4] = {64 * ((n + 127) / 128) + w128, 64 * ((n + 63) / 64) + (n + 63) / 64 * 64,
                                 64 * ((n + 31) / 32) + w32, 64 * ((n + 15) / 16) + w16};
        int best = 0;
        for (int i = 1; i < 4; i++)
            if (cost[i] < cost[best])
                best = i;
        // The residual stage takes 32 x 256 for the sixteen-fragment tiles
        // (launch_epi).
        if (best == 0 && !res)
            launch_epi<128, 128, 2, 2, KC, PW>(a, ob, rs, zw, s, res);
        else if (best == 1 && !res)
            launch_epi<64, 256, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
        else if (best <= 2)
            launch_epi<32, 256, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
        else
            launch_epi<16, 256, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
        return;
    }
    // Over few pixels a pointwise layer's 256-pixel tiles leave most CUs
    // idle (14 x 14 x 64 images: 49 tiles per channel block); 64-pixel tiles
    // give four times the workgroups, whose extra weight re-reads hit L2.
    const int64_t wgs_needed = 2 * int64_t(cu_count());
    auto few = [&](int64_t bc) { return PW && (int64_t(a.M) + 255) / 256 * ((n + bc - 1) / bc) < wgs_needed; };
    // The residual stage takes 64 x 64 or 32 x 256 for the sixteen-fragment
    // tiles (launch_epi).
    if (w128 <= w32 && w128 <= w16 && n > 64 && !res)
        launch_epi<128, 128, 2, 2, KC, PW>(a, ob, rs, zw, s, res);
    else if (w64 <= w32 && w64 <= w16 && n > 32 && (few(64) || !res)) {
        if (few(64))
            launch_epi<64, 64, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
        else
            launch_epi<64, 256, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
    } else if ((w32 <= w16 || res) && n > 16) {
        if (few(32))
            launch_epi<32, 64, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
        else
            launch_epi<32, 256, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
    } else {
        if (few(16))
            launch_epi<16, 64, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
        else
            launch_epi<16, 256, 1, 4, KC, PW>(a, ob, rs, zw, s, res);
    }
}

constexpr int HALO_LDS_MAX = 160 * 1024;  // LDS of one CU

template <int BC, int KC, int OB, bool RS, bool ZW>
void launch_halo(const HaloArgs& a, unsigned blocks, size_t lds, hipStream_t s)
{
    auto kfn = conv_i8_halo_kernel<BC, KC, OB, RS, ZW>;
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      HALO_LDS_MAX),
                  "conv_i8 halo LDS size");
        return true;
    }();
    (void)attr;
    hipLaunchKernelGGL(kfn, dim3(blocks, (a.N + BC - 1) / BC), dim3(HALO_NT), lds, s, a);
}

template <int BC, int KC>
void launch_halo_epi(const HaloArgs& a, unsigned blocks, size_t lds, int ob, bool rs, bool zw, hipStream_t s)
{
    if (!rs) {
        if (zw)
            launch_halo<BC, KC, 4, false, true>(a, blocks, lds, s);
        else
            launch_halo<BC, KC, 4, false, false>(a, blocks, lds, s);
        return;
    }
#define TOSA_HALO_OB(OBV)                                            \
    if (zw)                                                          \
        launch_halo<BC, KC, OBV, true, true>(a, blocks, lds, s);     \
    else                                                             \
        launch_halo<BC, KC, OBV, true, false>(a, blocks, lds, s);
    if (ob == 1) {
        TOSA_HALO_OB(1)
    } else if (ob == 2) {
        TOSA_HALO_OB(2)
    } else {
        TOSA_HALO_OB(4)
    }
#undef TOSA_HALO_OB
}

// Geometry of the halo kernel for `d`, or false when it does not apply:
// stride 1, ic a multiple of 64, output rows of at most 224 pixels with a
// tile that fills at least half of the 224-pixel workgroup tile, and a halo
// of at least 64 channels within the LDS budget.
bool halo_plan(const ConvI8Desc& d, bool zw, HaloArgs& a, int& bc, int& kc, size_t& lds, unsigned& blocks)
{
    if (d.sy != 1 || d.sx != 1 || d.ic % 64 != 0 || d.ow > HALO_BP || d.oh < 1 || d.ow < 1)
        return false;
    const int R = d.oh < HALO_BP / d.ow ? d.oh : HALO_BP / d.ow;
    if (2 * R * d.ow < HALO_BP)
        return false;
    const int HR = R + (d.kh - 1) * d.dy;
    const int HW = d.ow + (d.kw - 1) * d.dx;
    bc = d.oc > 64 ? 128 : 64;
    // LDS of a plan with `icc` halo channels: halo, NB weight stages, the
    // epilogue table and (nonzero weight zero point) the pixel sums.
    auto lds_for = [&](int icc) {
        const int k = icc % 128 == 0 ? 128 : 64;
        size_t b = size_t(HR) * HW * (icc + 16) + size_t(NB) * bc * k + size_t(32) * bc;
        if (zw)
            b += size_t(4) * (size_t(HR) * HW + HALO_BP);
        return b;
    };
    int icc = d.ic;
    while (icc >= 64 && (d.ic % icc != 0 || lds_for(icc) > size_t(HALO_LDS_MAX)))
        icc -= 64;
    if (icc < 64)
        return false;
    kc = icc % 128 == 0 ? 128 : 64;
    a.x = d.x;
    a.w = d.w;
    a.N = d.oc;
    a.K = d.kh * d.kw * d.ic;
    a.IC = d.ic;
    a.IH = d.ih;
    a.IW = d.iw;
    a.OH = d.oh;
    a.OW = d.ow;
    a.KH = d.kh;
    a.KW = d.kw;
    a.dy = d.dy;
    a.dx = d.dx;
    a.pt = d.pt;
    a.pl = d.pl;
    a.R = R;
    a.tiles_per_img = (d.oh + R - 1) / R;
    a.HR = HR;
    a.HW = HW;
    a.ICC = icc;
    a.ICS = icc + 16;
    a.halo_bytes = HR * HW * a.ICS;
    a.div_ow = FastDiv(uint32_t(d.ow));
    a.div_hw = FastDiv(uint32_t(HW));
    a.div_cpp = FastDiv(uint32_t(icc / 16));
    a.zp_x = d.zp_x;
    lds = lds_for(icc);
    blocks = unsigned(d.n) * unsigned(a.tiles_per_img);
    return true;
}

template <int BC, int PG, int TB, int KT, int OB, bool RS, bool ZW, int EL = HE_I8, int KP = 1>
void launch_halo32(const Halo32Args& a, unsigned blocks, size_t lds, hipStream_t s)
{
    auto kfn = conv_i8_halo32_kernel<EL, BC, PG, TB, KT, OB, RS, ZW, KP>;
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      HALO_LDS_MAX),
                  "conv_i8 halo32 LDS size");
        return true;
    }();
    (void)attr;
    hipLaunchKernelGGL(kfn, dim3(blocks, (a.N + BC - 1) / BC), dim3(BC / 64 * PG * 64), lds, s, a);
}

template <int BC, int PG, int TB, int KT, int KP = 1>
void launch_halo32_epi(const Halo32Args& a, unsigned blocks, size_t lds, int ob, bool rs, bool zw, hipStream_t s)
{
    if (!rs) {
        if (zw)
            launch_halo32<BC, PG, TB, KT, 4, false, true, HE_I8, KP>(a, blocks, lds, s);
        else
            launch_halo32<BC, PG, TB, KT, 4, false, false, HE_I8, KP>(a, blocks, lds, s);
        return;
    }
#define TOSA_HALO32_OB(OBV)                                                          \
    if (zw)                                                                          \
        launch_halo32<BC, PG, TB, KT, OBV, true, true, HE_I8, KP>(a, blocks, lds, s); \
    else                                                                             \
        launch_halo32<BC, PG, TB, KT, OBV, true, false, HE_I8, KP>(a, blocks, lds, s);
    if (ob == 1) {
        TOSA_HALO32_OB(1)
    } else if (ob == 2) {
        TOSA_HALO32_OB(2)
    } else {
        TOSA_HALO32_OB(4)
    }
#undef TOSA_HALO32_OB
}

}  // namespace

namespace {
std::atomic<int> g_conv_rows{1};
std::atomic<int> g_mm_rows{128};
}  // namespace

void set_mm_tile_rows(int rows) { g_mm_rows.store(rows == 64 ? 64 : 128); }
int mm_tile_rows() { return g_mm_rows.load(); }

void set_conv_rows_mode(int mode) { g_conv_rows.store(mode == 2 ? 2 : mode != 0); }
int conv_rows_mode() { return g_conv_rows.load(); }
bool conv_rows_enabled() { return g_conv_rows.load() != 0; }

// Compute units of the current device (workgroups of the 32x32 halo kernel
// that run at once: its LDS allows one per CU).
int cu_count()
{
    static int counts[64] = {0};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= 64)
        return 256;
    if (counts[dev] == 0) {
        int n = 0;
        hip_check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev), "CU count");
        counts[dev] = n > 0 ? n : 256;
    }
    return counts[dev];
}

namespace {

// Geometry of the 32x32 halo kernel for `d`, or false when it does not
// apply: stride 1, ic a multiple of 32, output rows of at most 512 pixels,
// tiles of at least 96 pixels and buffers within the LDS. Layouts (output
// channels x waves along the pixels x 32-pixel tiles per wave): 128 x 4 x 2,
// 64 x 8 x 2 and 64 x 8 x 1. Wave w sits on SIMD w % 4 and computes all
// its tiles when its first one holds pixels (none otherwise), so the
// busiest SIMD's MFMA work is the largest sum of its live waves' tiles. The
// layout and rows per tile R minimise (workgroup rounds, one workgroup per
// CU) x (that sum + 2), the 2 standing for a tile's fixed cost (first
// loads, epilogue); ties go to the fewest bytes loaded per CU (weights +
// halo: the loads' issue holds up the waves that make them).
bool halo32_plan(const ConvI8Desc& d, bool zw, Halo32Args& a, int& bc, size_t& lds, unsigned& blocks,
                 bool allow_kp2 = true)
{
    if (d.sy != 1 || d.sx != 1 || d.ic % 32 != 0 || d.ow > H32_BP_MAX || d.oh < 1 || d.ow < 1 || d.depthwise)
        return false;
    const int taps = d.kh * d.kw;
    const int HW = d.ow + (d.kw - 1) * d.dx;
    auto lds_for = [&](int R, int c, int bp, int kp = 1) {
        const size_t hw = (size_t(R) + size_t(d.kh - 1) * d.dy) * HW;
        size_t b = 2 * ((hw * 64 + 1023) / 1024 * 1024) + 2 * size_t(kp) * taps * c * 32 + size_t(32) * c;
        if (zw)
            b += size_t(4) * (hw + bp);
        return b;
    };
    const long cus = cu_count();
    int R = 0, PG = 0, TB = 0;
    bc = 0;
    long best = 0, best_bytes = 0;
    const int layouts[3][3] = {{128, 4, 2}, {64, 8, 2}, {64, 8, 1}};
    for (const auto& lay : layouts) {
        const int c = lay[0], pg = lay[1], tb = lay[2], bp = h32_bp(pg, tb);
        if ((c == 128 && d.oc <= 64) || d.ow > bp)
            continue;
        const int rmax = d.oh < bp / d.ow ? d.oh : bp / d.ow;
        const long chb = (d.oc + c - 1) / c;
        for (int r = rmax; r >= 1; r--) {
            if (r * d.ow < 96 && r != d.oh)
                break;
            if (lds_for(r, c, bp) > size_t(HALO_LDS_MAX))
                continue;
            const int tiles = (r * d.ow + 31) / 32;
            long simd_max = 0;
            for (int sm = 0; sm < 4; sm++) {
                long t = 0;
                for (int w = sm; w < c / 64 * pg; w += 4)
                    t += (w % pg) < tiles ? tb : 0;
                simd_max = t > simd_max ? t : simd_max;
            }
            const long nb = long(d.n) * ((d.oh + r - 1) / r) * chb;
            const long rounds = (nb + cus - 1) / cus;
            const long cost = rounds * (simd_max + 2);
            const long bytes = rounds * (long(taps) * c * d.ic + (long(r) + long(d.kh - 1) * d.dy) * HW * d.ic);
            if (R == 0 || cost < best || (cost == best && bytes < best_bytes)) {
                R = r;
                PG = pg;
                TB = tb;
                bc = c;
                best = cost;
                best_bytes = bytes;
            }
        }
    }
    if (R == 0 || R * d.ow < 96)
        return false;
    a.x = d.x;
    a.wp = d.wpack;
    a.N = d.oc;
    a.IC = d.ic;
    a.IH = d.ih;
    a.IW = d.iw;
    a.OH = d.oh;
    a.OW = d.ow;
    a.KW = d.kw;
    a.taps = taps;
    a.dy = d.dy;
    a.dx = d.dx;
    a.pt = d.pt;
    a.pl = d.pl;
    a.R = R;
    a.tiles_per_img = (d.oh + R - 1) / R;
    a.HR = R + (d.kh - 1) * d.dy;
    a.HW = HW;
    a.sbytes = int32_t((size_t(a.HR) * HW * 64 + 1023) / 1024 * 1024);
    a.wbytes = taps * bc * 32;
    a.PG = PG;
    a.TB = TB;
    // Whole 64-byte stages per pass where the kernel has that variant (the
    // 64-channel two-tile layout, 3x3 taps) and the doubled weight buffer
    // fits.
    a.KP = allow_kp2 && bc == 64 && PG == 8 && TB == 2 && taps == 9 && d.ic % 64 == 0 &&
                   lds_for(R, bc, h32_bp(PG, TB), 2) <= size_t(HALO_LDS_MAX)
               ? 2
               : 1;
    a.div_ow = FastDiv(uint32_t(d.ow));
    a.div_hw = FastDiv(uint32_t(HW));
    lds = lds_for(R, bc, h32_bp(PG, TB), a.KP);
    blocks = unsigned(d.n) * unsigned(a.tiles_per_img);
    return true;
}

// Geometry of the row-tile kernel for `d`, or false when it does not apply:
// a 3x3 stride-1 undilated CONV2D with 128 input channels, output rows of
// 17-30 pixels, output channels a multiple of 64 and no weight zero point
// (one workgroup per CU). CB: 32-channel blocks per workgroup (4 when the
// channels allow, else 2 and two producer waves along the rows).
bool rows_plan(const ConvI8Desc& d, RowsArgs& a, int& cb, size_t& lds, unsigned& blocks)
{
    if (!conv_rows_enabled() || d.depthwise || d.kh != 3 || d.kw != 3 || d.sy != 1 || d.sx != 1 || d.dy != 1 ||
        d.dx != 1 || d.zp_w != 0 || d.ic != 128 || d.ow < 17 || d.ow > ROWS_HWP - 2 || d.oc % 64 != 0 ||
        d.batch != 1)
        return false;
    cb = d.oc % 128 == 0 && conv_rows_mode() != 2 ? 4 : 2;
    const int rows = 4 / cb * ROWS_RW;
    a.x = d.x;
    a.wp = d.wpack;
    a.N = d.oc;
    a.IC = d.ic;
    a.IH = d.ih;
    a.IW = d.iw;
    a.OH = d.oh;
    a.OW = d.ow;
    a.pt = d.pt;
    a.pl = d.pl;
    a.row_tiles = (d.oh + rows - 1) / rows;
    a.ch_tiles = d.oc / (32 * cb);
    lds = rows_lds(cb);
    const int64_t nb = int64_t(d.n) * a.row_tiles * a.ch_tiles;
    if (nb >= (int64_t(1) << 31))
        return false;
    blocks = unsigned(nb);
    return true;
}

template <int CB, int OB, bool RS, bool RC>
void launch_rows(const RowsArgs& a, unsigned blocks, size_t lds, hipStream_t s)
{
    auto kfn = conv_i8_rows_kernel<4, CB, OB, RS, RC>;
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      HALO_LDS_MAX),
                  "conv_i8 rows LDS size");
        return true;
    }();
    (void)attr;
    if (lds > size_t(HALO_LDS_MAX))
        throw std::runtime_error("conv_i8 rows: LDS image too large");
    hipLaunchKernelGGL(kfn, dim3(blocks), dim3(512), lds, s, a);
}

template <int CB>
void launch_rows_epi(const RowsArgs& a, unsigned blocks, size_t lds, int ob, bool rs, bool rc, hipStream_t s)
{
    if (!rs)
        launch_rows<CB, 4, false, false>(a, blocks, lds, s);
    else if (ob == 1)
        rc ? launch_rows<CB, 1, true, true>(a, blocks, lds, s) : launch_rows<CB, 1, true, false>(a, blocks, lds, s);
    else if (ob == 2)
        rc ? launch_rows<CB, 2, true, true>(a, blocks, lds, s) : launch_rows<CB, 2, true, false>(a, blocks, lds, s);
    else
        rc ? launch_rows<CB, 4, true, true>(a, blocks, lds, s) : launch_rows<CB, 4, true, false>(a, blocks, lds, s);
}

template <int G, int OB, bool RS, bool ZW>
void launch_dw(const DwArgs& a, hipStream_t s)
{
    const int64_t items = int64_t((a.P + 63) / 64) * (a.C / 16);
    hipLaunchKernelGGL((conv_i8_dw_kernel<G, OB, RS, ZW>), dim3(unsigned((items + 3) / 4)), dim3(256), 0, s, a);
}

template <int G>
void launch_dw_epi(const DwArgs& a, int ob, bool rs, bool zw, hipStream_t s)
{
    if (!rs) {
        if (zw)
            launch_dw<G, 4, false, true>(a, s);
        else
            launch_dw<G, 4, false, false>(a, s);
        return;
    }
#define TOSA_DW_OB(OBV)                          \
    if (zw)                                      \
        launch_dw<G, OBV, true, true>(a, s);     \
    else                                         \
        launch_dw<G, OBV, true, false>(a, s);
    if (ob == 1) {
        TOSA_DW_OB(1)
    } else if (ob == 2) {
        TOSA_DW_OB(2)
    } else {
        TOSA_DW_OB(4)
    }
#undef TOSA_DW_OB
}

}  // namespace

namespace {
// Residual constants of channel c: for each of RESCALE(y), RESCALE(skip)
// and the final RESCALE, {m, s, rp (2 words), rn (2 words)} with the
// sign-selected rounding constants of apply_scale_32 (the last one carrying
// its output zero point), then -2^min(s - 1, 31) of the final RESCALE.
__global__ void conv_i8_residual_table_kernel(RescaleDev ra, RescaleDev rb, RescaleDev ro, int32_t channels,
                                              int32_t* out)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= channels)
        return;
    int32_t* q = out + int64_t(c) * CONV_I8_RES_WORDS;
    auto put = [&](const RescaleDev& r, int64_t zp, int32_t* w) {
        const int ch = r.per_channel ? c : 0;
        const int32_t m = r.mult[ch], s = r.shift[ch];
        const int64_t half = int64_t(1) << (s - 1);
        const int64_t d = (r.rounding == 3 && s > 31) ? (int64_t(1) << 30) : 0;
        const int64_t z = zp * (int64_t(1) << s);
        const int64_t rp = half + d + z, rn = half - d + z;
        w[0] = m;
        w[1] = s;
        w[2] = int32_t(uint64_t(rp));
        w[3] = int32_t(uint64_t(rp) >> 32);
        w[4] = int32_t(uint64_t(rn));
        w[5] = int32_t(uint64_t(rn) >> 32);
        return s;
    };
    put(ra, 0, q);
    put(rb, 0, q + 6);
    const int32_t so = put(ro, ro.out_zp, q + 12);
    q[18] = so - 1 < 31 ? -(int32_t(1) << (so - 1)) : INT32_MIN;
    q[19] = 0;
}
}  // namespace

void conv_i8_residual_table(const RescaleDev& ra, const RescaleDev& rb, const RescaleDev& ro, int32_t channels,
                            void* out, hipStream_t stream)
{
    if (channels <= 0)
        return;
    hipLaunchKernelGGL(conv_i8_residual_table_kernel, dim3(unsigned((channels + 255) / 256)), dim3(256), 0, stream,
                       ra, rb, ro, channels, static_cast<int32_t*>(out));
}

bool conv_i8_residual_ok(const ConvI8Desc& d, const RescaleDev& rs, const RescaleDev& ra, const RescaleDev& rb,
                         const RescaleDev& ro, const void* skip)
{
    const bool pw = !d.depthwise && d.kh == 1 && d.kw == 1 && d.sy == 1 && d.sx == 1 && d.pt == 0 && d.pl == 0 &&
                    d.ih == d.oh && d.iw == d.ow;
    const int64_t ch = d.oc;
    // The input RESCALEs: int8 -> int32, SINGLE/DOUBLE rounding, shifts >= 9
    // (|x - zp| <= 255 < 2^(s-1): the range REQUIRE holds, and the scaled
    // value fits int32), no output zero point or CLAMP.
    auto in_ok = [ch](const RescaleDev& r) {
        return r.scale32 && (r.rounding == 1 || r.rounding == 3) && r.in_bits == 8 && !r.in_unsigned &&
               r.out_bytes == 4 && r.out_zp == 0 && !r.has_clamp && r.min_shift >= 9 &&
               (!r.per_channel || r.channels == ch);
    };
    // The final RESCALE: int32 -> int8 with an output zero point the
    // rounding constants can carry (|zp| 2^s <= 2^60).
    const int64_t zp = ro.out_zp < 0 ? -ro.out_zp : ro.out_zp;
    const bool fold = zp == 0 || (ro.max_shift <= 60 && zp <= (int64_t(1) << (60 - ro.max_shift)));
    const bool o_ok = ro.scale32 && (ro.rounding == 1 || ro.rounding == 3) && ro.in_bits == 32 && !ro.in_unsigned &&
                      ro.in_zp == 0 && ro.out_bytes == 1 && fold && (!ro.per_channel || ro.channels == ch);
    // The convolution's own RESCALE gives int8 without a CLAMP.
    const bool y_ok = conv_i8_fast_epilogue_ok(rs) && rs.out_bytes == 1 && !rs.has_clamp && rs.lo == -128 &&
                      rs.hi == 127;
    return pw && d.batch == 1 && conv_i8_fast_supported(d) && y_ok && in_ok(ra) && in_ok(rb) && o_ok &&
           ch % 4 == 0 && ch <= 1024 && reinterpret_cast<uintptr_t>(skip) % 4 == 0;
}

bool matmul_i8_direct_applies(int32_t C, int32_t W, const void* a, const void* b)
{
    return C >= 128 && C % 128 == 0 && W >= 16 && W % 16 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(b) % 16 == 0;
}

namespace {
template <int OB, bool RS, bool ZA, bool ZB, bool RC>
void launch_mm(const MatmulI8Args& a, int32_t batch, int rows, hipStream_t s)
{
    auto go = [&](auto wpc) {
        constexpr int WP = decltype(wpc)::value;
        auto kfn = matmul_i8_kernel<WP, OB, RS, ZA, ZB, RC>;
        static bool attr = [&]() {
            hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn),
                                          hipFuncAttributeMaxDynamicSharedMemorySize, int(mm_lds(WP))),
                      "matmul_i8 LDS size");
            return true;
        }();
        (void)attr;
        hipLaunchKernelGGL(kfn, dim3(unsigned(int64_t(a.HT) * a.WT * batch)), dim3(128 * WP), mm_lds(WP), s, a);
    };
    if (rows == mm_bh(4))
        go(std::integral_constant<int, 4>{});
    else
        go(std::integral_constant<int, 2>{});
}
template <int OB, bool RS, bool RC>
void launch_mm_zp(const MatmulI8Args& a, int32_t batch, int rows, bool za, bool zb, hipStream_t s)
{
    if (za)
        zb ? launch_mm<OB, RS, true, true, RC>(a, batch, rows, s) : launch_mm<OB, RS, true, false, RC>(a, batch, rows, s);
    else
        zb ? launch_mm<OB, RS, false, true, RC>(a, batch, rows, s) : launch_mm<OB, RS, false, false, RC>(a, batch, rows, s);
}
}  // namespace

bool matmul_i8_direct(const int8_t* a, const int8_t* b, int32_t batch, int32_t H, int32_t C, int32_t W, int32_t zp_a,
                      int32_t zp_b, const void* tab, const RescaleDev* rs, bool range_safe, void* out, uint32_t* err,
                      hipStream_t stream)
{
    // The kernel addresses a batch's rows of A, and a stage's 128 rows of B,
    // with 32-bit offsets.
    if (!matmul_i8_direct_applies(C, W, a, b) || (rs && !conv_i8_fast_epilogue_ok(*rs)) ||
        int64_t(H) * C >= (int64_t(1) << 31) || int64_t(W) * MM_KC >= (int64_t(1) << 31))
        return false;
    if (int64_t(batch) * H <= 0)
        return true;
    MatmulI8Args m{};
    m.a = a;
    m.b = b;
    m.tab = static_cast<const v4i*>(tab);
    m.H = H;
    m.C = C;
    m.W = W;
    const int rows = mm_tile_rows();  // read once: HT and the launch agree
    m.HT = (H + rows - 1) / rows;
    m.WT = (W + 127) / 128;
    m.batch = batch;
    if (int64_t(m.HT) * m.WT * batch >= (int64_t(1) << 31))
        return false;
    m.zp_a = zp_a;
    EpiArgs& e = m.E;
    e.out = static_cast<uint8_t*>(out);
    e.N = W;
    e.zp_w = zp_b;
    e.err = err;
    int ob = 4;
    if (rs) {
        e.clo = int32_t(rs->has_clamp ? std::max<int64_t>(rs->clamp_lo, rs->lo) : rs->lo);
        e.chi = int32_t(rs->has_clamp ? std::min<int64_t>(rs->clamp_hi, rs->hi) : rs->hi);
        e.range = rs->min_shift <= 31 && !range_safe;
        e.one_round = rs->rounding != 3 || rs->max_shift <= 31;
        ob = rs->out_bytes;
    }
    const bool za = zp_a != 0, zb = zp_b != 0;
    if (!rs)
        launch_mm_zp<4, false, false>(m, batch, rows, za, zb, stream);
    else if (e.range)
        ob == 1 ? launch_mm_zp<1, true, true>(m, batch, rows, za, zb, stream)
                : ob == 2 ? launch_mm_zp<2, true, true>(m, batch, rows, za, zb, stream)
                          : launch_mm_zp<4, true, true>(m, batch, rows, za, zb, stream);
    else
        ob == 1 ? launch_mm_zp<1, true, false>(m, batch, rows, za, zb, stream)
                : ob == 2 ? launch_mm_zp<2, true, false>(m, batch, rows, za, zb, stream)
                          : launch_mm_zp<4, true, false>(m, batch, rows, za, zb, stream);
    return true;
}

bool conv_i8_pointwise_stream(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                              hipStream_t stream)
{
    const bool pw = !d.depthwise && d.kh == 1 && d.kw == 1 && d.sy == 1 && d.sx == 1 && d.pt == 0 && d.pl == 0 &&
                    d.ih == d.oh && d.iw == d.ow;
    if (!rs || !conv_i8_fast_epilogue_ok(*rs) || !pws_applies(d, pw, rs->out_bytes, rs))
        return false;
    PwsArgs a{};
    a.x = d.x;
    a.w = d.w;
    a.tab = static_cast<const v4i*>(tab);
    a.M = d.n * d.oh * d.ow;
    a.K = d.ic;
    a.N = d.oc;
    a.ntiles = (a.M + 31) / 32;
    EpiArgs& e = a.E;
    e.out = static_cast<uint8_t*>(out);
    e.N = d.oc;
    e.zp_w = d.zp_w;
    e.err = err;
    e.clo = int32_t(rs->has_clamp ? std::max<int64_t>(rs->clamp_lo, rs->lo) : rs->lo);
    e.chi = int32_t(rs->has_clamp ? std::min<int64_t>(rs->clamp_hi, rs->hi) : rs->hi);
    e.range = rs->min_shift <= 31 && !d.range_safe;
    e.one_round = rs->rounding != 3 || rs->max_shift <= 31;
    const bool zw = d.zp_w != 0;
    if (d.ic <= 32) {
        if (zw)
            launch_pws_ta<1, true>(a, stream);
        else
            launch_pws_ta<1, false>(a, stream);
    } else {
        if (zw)
            launch_pws_ta<2, true>(a, stream);
        else
            launch_pws_ta<2, false>(a, stream);
    }
    return true;
}

bool conv_i8_stem(const ConvI8Desc& d, const void* tab, const int8_t* wpad, const RescaleDev* rs, void* out,
                  uint32_t* err, hipStream_t stream)
{
    if (!rs || rs->out_bytes != 1 || !conv_i8_fast_epilogue_ok(*rs) || d.depthwise || d.batch != 1 || d.ic != 3 ||
        d.kh != 3 || d.kw != 3 || d.dy != 1 || d.dx != 1 || d.iw % 4 != 0 || d.sy < 1 || d.sy > 2 || d.sx < 1 ||
        d.sx > 2 || d.pt < 0 || d.pt > 2 || d.pl < 0 || d.pl > 2 || d.oc % 32 != 0 ||
        reinterpret_cast<uintptr_t>(d.x) % 4 != 0 || reinterpret_cast<uintptr_t>(wpad) % 16 != 0 ||
        int64_t(d.n) * d.oh * d.ow < 4096 || int64_t(d.n) * d.ih * d.iw * 3 >= (int64_t(1) << 31))
        return false;
    StemArgs a{};
    a.WP = (d.ow - 1) * d.sx + 3;
    if (a.WP < d.pl + d.iw)
        return false;  // the image's own columns must all be staged
    a.x = d.x;
    a.w = wpad;
    a.tab = static_cast<const v4i*>(tab);
    a.N = d.oc;
    a.IH = d.ih;
    a.IW = d.iw;
    a.OH = d.oh;
    a.OW = d.ow;
    a.sy = d.sy;
    a.sx = d.sx;
    a.pt = d.pt;
    a.pl = d.pl;
    // Rows per band: staged rows within 32 KB of LDS, and bands enough for
    // four workgroups per CU.
    int R = std::max(1, std::min(d.oh, ((32 * 1024) / (4 * a.WP) - 3) / d.sy + 1));
    while (R > 1 && int64_t(d.n) * ((d.oh + R - 1) / R) < 4 * int64_t(cu_count()))
        R = (R + 1) / 2;
    a.R = R;
    a.bands = (d.oh + R - 1) / R;
    a.units = d.n * a.bands;
    a.HR = (R - 1) * d.sy + 3;
    a.zfw = (uint32_t(uint8_t(d.zp_x)) * 0x010101u);
    a.div_ow = FastDiv(uint32_t(d.ow));
    a.div_bands = FastDiv(uint32_t(a.bands));
    a.div_g = FastDiv(uint32_t(d.iw / 4));
    EpiArgs& e = a.E;
    e.out = static_cast<uint8_t*>(out);
    e.N = d.oc;
    e.zp_w = d.zp_w;
    e.err = err;
    e.clo = int32_t(rs->has_clamp ? std::max<int64_t>(rs->clamp_lo, rs->lo) : rs->lo);
    e.chi = int32_t(rs->has_clamp ? std::min<int64_t>(rs->clamp_hi, rs->hi) : rs->hi);
    e.range = rs->min_shift <= 31 && !d.range_safe;
    e.one_round = rs->rounding != 3 || rs->max_shift <= 31;
    const size_t lds = size_t(a.HR) * a.WP * 4;
    if (lds > 64 * 1024)
        return false;
    const dim3 grid(unsigned(a.units), unsigned(d.oc / 32));
    if (d.zp_w != 0)
        hipLaunchKernelGGL(conv_i8_stem_kernel<true>, grid, dim3(256), lds, stream, a);
    else
        hipLaunchKernelGGL(conv_i8_stem_kernel<false>, grid, dim3(256), lds, stream, a);
    return true;
}

bool conv_i8_fast_supported(const ConvI8Desc& d)
{
    if (d.depthwise)
        return d.ic % 16 == 0 && d.oc == d.ic && d.kh * d.kw <= 12 && reinterpret_cast<uintptr_t>(d.x) % 16 == 0;
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
    // Weight element (channel c, reduction index k): OHWI w[c K + k]; depthwise
    // [KH, KW, C, 1] w[k C + c].
    const int32_t K = d.depthwise ? d.kh * d.kw : d.kh * d.kw * d.ic;
    const int32_t cstride = d.depthwise ? 1 : K, kstride = d.depthwise ? d.ic : 1;
    const int batch = d.depthwise ? 1 : d.batch;
    hipLaunchKernelGGL(conv_i8_table_kernel, dim3(d.oc, batch), dim3(64), 0, stream, d.w, d.oc, K, cstride, kstride,
                       d.bias, d.bias_len, d.zp_x, d.zp_w, rs ? rs->mult : nullptr, rs ? rs->shift : nullptr,
                       rs ? rs->per_channel : 0, rs ? int32_t(rs->rounding == 3) : 0,
                       rs ? int32_t(rs->out_zp) : 0, static_cast<v4i*>(tab), int64_t(d.oc) * K,
                       int32_t(conv_i8_table_stride(d.oc) / 4));
}

bool conv_i8_table_range_safe(const ConvI8Desc& d, const void* tab)
{
    if (d.oc <= 0)
        return true;
    const int batch = d.depthwise ? 1 : d.batch;
    std::vector<int32_t> h(size_t(conv_i8_table_words(d.oc, batch)));
    hip_check(hipMemcpy(h.data(), tab, h.size() * sizeof(int32_t), hipMemcpyDeviceToHost), "conv_i8 table readback");
    const int64_t stride = conv_i8_table_stride(d.oc);
    for (int b = 0; b < batch; b++)
        for (int c = 0; c < d.oc; c++)
            if (h[size_t(b * stride + int64_t(CONV_I8_TABLE_WORDS) * c + 2)] != INT32_MIN)
                return false;
    return true;
}

int32_t conv_i8_im2col_kp(const ConvI8Desc& d) { return (d.kh * d.kw * d.ic + 15) / 16 * 16; }

void conv_i8_im2col(const ConvI8Desc& d, int8_t* xcol, hipStream_t stream)
{
    Im2colArgs a{};
    a.x = d.x;
    a.out = xcol;
    a.M = d.n * d.oh * d.ow;
    a.K = d.kh * d.kw * d.ic;
    a.Kp = conv_i8_im2col_kp(d);
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
    if (a.M <= 0)
        return;
    const dim3 grid(unsigned((a.M + 255) / 256), unsigned(a.Kp / 16));
    if (a.Kp <= IM2COL_TAB) {
        Im2colTab t{};
        for (int k = 0; k < a.Kp; k++) {
            if (k >= a.K) {
                t.off[k] = -1;
                continue;
            }
            const int tap = k / d.ic, ic = k % d.ic;
            const int ky = tap / d.kw, kx = tap % d.kw;
            t.dy[k] = int16_t(ky * d.dy);
            t.dx[k] = int16_t(kx * d.dx);
            t.off[k] = (ky * d.dy * d.iw + kx * d.dx) * d.ic + ic;
        }
        if (d.ic % 4 == 0 && reinterpret_cast<uintptr_t>(d.x) % 4 == 0)
            hipLaunchKernelGGL(conv_i8_im2col_tab_kernel<true>, grid, dim3(256), 0, stream, a, t);
        else
            hipLaunchKernelGGL(conv_i8_im2col_tab_kernel<false>, grid, dim3(256), 0, stream, a, t);
        return;
    }
    hipLaunchKernelGGL(conv_i8_im2col_kernel, grid, dim3(256), 0, stream, a);
}

void conv_i8_rowpad(const int8_t* w, int32_t rows, int32_t k, int32_t kp, int8_t* out, hipStream_t stream)
{
    const int64_t n = int64_t(rows) * kp;
    if (n <= 0)
        return;
    hipLaunchKernelGGL(conv_i8_rowpad_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, w, rows, k, kp,
                       out);
}

void transpose_b_i8(const int8_t* b, int32_t batch, int32_t c, int32_t w, int8_t* out, hipStream_t stream)
{
    if (int64_t(batch) * c * w <= 0)
        return;
    const dim3 grid(unsigned((w + 64 * TR_TT - 1) / (64 * TR_TT)), unsigned((c + 63) / 64), unsigned(batch));
    if (w % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0)
        hipLaunchKernelGGL(transpose_b_kernel<true>, grid, dim3(256), 0, stream, b, c, w, out);
    else
        hipLaunchKernelGGL(transpose_b_kernel<false>, grid, dim3(256), 0, stream, b, c, w, out);
}

// Channel block of the packed weights (the halo kernel's workgroup
// channels), 0 when the halo kernel does not run for `d`.
int conv_i8_wpack_block(const ConvI8Desc& d)
{
    Halo32Args a{};
    int bc = 0;
    size_t lds = 0;
    unsigned blocks = 0;
    const bool pw = d.kh == 1 && d.kw == 1 && d.sy == 1 && d.sx == 1 && d.pt == 0 && d.pl == 0 && d.ih == d.oh &&
                    d.iw == d.ow;
    if (pw || !conv_i8_fast_supported(d))
        return 0;
    RowsArgs ra{};
    int cb = 0;
    if (rows_plan(d, ra, cb, lds, blocks))
        return 32;
    if (!halo32_plan(d, d.zp_w != 0, a, bc, lds, blocks))
        return 0;
    return bc;
}

int64_t conv_i8_wpack_bytes(const ConvI8Desc& d)
{
    const int bc = conv_i8_wpack_block(d);
    if (bc == 0)
        return 0;
    return int64_t((d.oc + bc - 1) / bc) * bc * d.kh * d.kw * d.ic;
}

void conv_i8_wpack(const ConvI8Desc& d, void* wp, hipStream_t stream)
{
    const int64_t bytes = conv_i8_wpack_bytes(d);
    if (bytes <= 0)
        return;
    const int bc = conv_i8_wpack_block(d);
    const int64_t slots = bytes / 16;
    hipLaunchKernelGGL(conv_i8_wpack_kernel, dim3(unsigned((slots + 255) / 256)), dim3(256), 0, stream, d.w, d.oc,
                       d.kh * d.kw * d.ic, d.ic, d.kh * d.kw, bc, slots, static_cast<v4u*>(wp));
}

bool conv_i8_fast_epilogue_ok(const RescaleDev& rs)
{
    // The table folds the output zero point into the rounding constants,
    // exact while |zp| 2^max_shift <= 2^60 keeps the 64-bit sum in range;
    // every legal zero point (int8, uint8, uint16, or 0 for int32) with a
    // shift up to 45 qualifies. The sum r + zp then fits int32 (|r| <=
    // 2^30 + 1), so RESCALE's int32 check cannot fail.
    const int64_t zp = rs.out_zp < 0 ? -rs.out_zp : rs.out_zp;
    const bool fold = zp == 0 || (rs.max_shift >= 2 && rs.max_shift <= 60 && zp <= (int64_t(1) << (60 - rs.max_shift)));
    return rs.scale32 && (rs.rounding == 1 || rs.rounding == 3) && !rs.in_unsigned && rs.in_zp == 0 &&
           (rs.out_bytes == 1 || rs.out_bytes == 2 || rs.out_bytes == 4) && fold;
}

void conv_i8_fast(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                  hipStream_t stream)
{
    EpiArgs e{};
    e.out = static_cast<uint8_t*>(out);
    e.N = d.oc;
    e.zp_w = d.zp_w;
    e.err = err;
    int ob = 4;
    if (rs) {
        // CLAMP bounds are values of the output type, so they lie inside
        // [lo, hi] (prepare_clamp_int decodes them in that type).
        e.clo = int32_t(rs->has_clamp ? std::max<int64_t>(rs->clamp_lo, rs->lo) : rs->lo);
        e.chi = int32_t(rs->has_clamp ? std::min<int64_t>(rs->clamp_hi, rs->hi) : rs->hi);
        e.range = rs->min_shift <= 31 && !d.range_safe;
        e.one_round = rs->rounding != 3 || rs->max_shift <= 31;
        ob = rs->out_bytes;
    }
    if (int64_t(d.n) * d.oh * d.ow <= 0 || d.oc <= 0)
        return;
    const bool zw = d.zp_w != 0;
    if (d.depthwise && (depthwise_i8_pipe(d, tab, rs, out, err, stream) || depthwise_i8_lds(d, tab, rs, out, err, stream)))
        return;
    if (d.depthwise) {
        DwArgs w{};
        w.x = d.x;
        w.w = d.w;
        w.tab = static_cast<const v4i*>(tab);
        w.P = d.n * d.oh * d.ow;
        w.C = d.ic;
        w.IH = d.ih;
        w.IW = d.iw;
        w.OH = d.oh;
        w.OW = d.ow;
        w.KW = d.kw;
        w.T = d.kh * d.kw;
        w.sy = d.sy;
        w.sx = d.sx;
        w.dy = d.dy;
        w.dx = d.dx;
        w.pt = d.pt;
        w.pl = d.pl;
        w.div_ohow = FastDiv(uint32_t(d.oh * d.ow));
        w.div_ow = FastDiv(uint32_t(d.ow));
        w.zp_x = d.zp_x;
        w.E = e;
        const int groups = (w.T + 3) / 4;
        if (groups == 1)
            launch_dw_epi<1>(w, ob, rs != nullptr, zw, stream);
        else if (groups == 2)
            launch_dw_epi<2>(w, ob, rs != nullptr, zw, stream);
        else
            launch_dw_epi<3>(w, ob, rs != nullptr, zw, stream);
        return;
    }
    const bool pw = d.kh == 1 && d.kw == 1 && d.sy == 1 && d.sx == 1 && d.pt == 0 && d.pl == 0 && d.ih == d.oh &&
                    d.iw == d.ow;
    const bool res = d.res_skip != nullptr;
    if (res) {
        e.skip = d.res_skip;
        e.za = d.res_za;
        e.zb = d.res_zb;
        e.rclo = d.res_clo;
        e.rchi = d.res_chi;
    }
    if (!res && pws_applies(d, pw, ob, rs)) {
        PwsArgs a{};
        a.x = d.x;
        a.w = d.w;
        a.tab = static_cast<const v4i*>(tab);
        a.M = d.n * d.oh * d.ow;
        a.K = d.ic;
        a.N = d.oc;
        a.ntiles = (a.M + 31) / 32;
        a.E = e;
        if (d.ic <= 32) {
            if (zw)
                launch_pws_ta<1, true>(a, stream);
            else
                launch_pws_ta<1, false>(a, stream);
        } else {
            if (zw)
                launch_pws_ta<2, true>(a, stream);
            else
                launch_pws_ta<2, false>(a, stream);
        }
        return;
    }

    int bc = 128, kc = 128;
    size_t lds = 0;
    unsigned blocks = 0;
    RowsArgs ra{};
    int cb = 0;
    if (!pw && d.wpack && rows_plan(d, ra, cb, lds, blocks)) {
        ra.tab = static_cast<const v4i*>(tab);
        ra.zfill = reinterpret_cast<const int8_t*>(ra.tab + 2 * d.oc);
        ra.E = e;
        if (cb == 4)
            launch_rows_epi<4>(ra, blocks, lds, ob, rs != nullptr, e.range != 0, stream);
        else
            launch_rows_epi<2>(ra, blocks, lds, ob, rs != nullptr, e.range != 0, stream);
        return;
    }
    Halo32Args h32{};
    if (!pw && d.wpack && halo32_plan(d, zw, h32, bc, lds, blocks)) {
        h32.tab = static_cast<const v4i*>(tab);
        h32.zfill = reinterpret_cast<const int8_t*>(h32.tab + 2 * d.oc);
        h32.E = e;
        const bool k3 = d.kh == 3 && d.kw == 3;
        if (bc == 128) {
            if (k3)
                launch_halo32_epi<128, 4, 2, 9>(h32, blocks, lds, ob, rs != nullptr, zw, stream);
            else
                launch_halo32_epi<128, 4, 2, 0>(h32, blocks, lds, ob, rs != nullptr, zw, stream);
        } else if (h32.TB == 2) {
            if (k3 && h32.KP == 2)
                launch_halo32_epi<64, 8, 2, 9, 2>(h32, blocks, lds, ob, rs != nullptr, zw, stream);
            else if (k3)
                launch_halo32_epi<64, 8, 2, 9>(h32, blocks, lds, ob, rs != nullptr, zw, stream);
            else
                launch_halo32_epi<64, 8, 2, 0>(h32, blocks, lds, ob, rs != nullptr, zw, stream);
        } else {
            if (k3)
                launch_halo32_epi<64, 8, 1, 9>(h32, blocks, lds, ob, rs != nullptr, zw, stream);
            else
                launch_halo32_epi<64, 8, 1, 0>(h32, blocks, lds, ob, rs != nullptr, zw, stream);
        }
        return;
    }
    HaloArgs h{};
    if (!pw && halo_plan(d, zw, h, bc, kc, lds, blocks)) {
        h.tab = static_cast<const v4i*>(tab);
        h.E = e;
        if (bc == 128) {
            if (kc == 128)
                launch_halo_epi<128, 128>(h, blocks, lds, ob, rs != nullptr, zw, stream);
            else
                launch_halo_epi<128, 64>(h, blocks, lds, ob, rs != nullptr, zw, stream);
        } else {
            if (kc == 128)
                launch_halo_epi<64, 128>(h, blocks, lds, ob, rs != nullptr, zw, stream);
            else
                launch_halo_epi<64, 64>(h, blocks, lds, ob, rs != nullptr, zw, stream);
        }
        return;
    }

    ConvI8Args a{};
    a.x = d.x;
    a.w = d.w;
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
    a.E = e;
    a.batch = pw ? d.batch : 1;
    a.bsx = int64_t(a.M) * a.K;
    a.bsw = int64_t(a.N) * a.K;
    a.bso = int64_t(a.M) * a.N * ob;
    a.bst = int32_t(conv_i8_table_stride(d.oc) / 4);
    if (pw) {
        // 128-byte reduction steps, except for 128 < K < 192, where 64-byte
        // ones stage a quarter fewer bytes (K = 144: 192 per row instead of
        // 256; 144 -> 24 at 56 x 56: 18.3 -> 13.6 us). For longer K the extra
        // steps cost more than the padding (K = 960 over 7 x 7 images: 3-4 us
        // slower with 64).
        a.rtab = static_cast<const int32_t*>(d.res_tab);
        if (a.K >= 192 || a.K == 128)
            launch_tile<128, true>(a, ob, rs != nullptr, zw, stream, res);
        else
            launch_tile<64, true>(a, ob, rs != nullptr, zw, stream, res);
    } else if (d.ic % 128 == 0) {
        launch_tile<128, false>(a, ob, rs != nullptr, zw, stream);
    } else {
        launch_tile<64, false>(a, ob, rs != nullptr, zw, stream);
    }
}

namespace {

// The byte view of a float convolution that the halo planner and weight
// packing take: every channel is two bytes.
ConvI8Desc f16_byte_desc(const ConvF16Desc& d)
{
    ConvI8Desc b;
    b.x = static_cast<const int8_t*>(d.x);
    b.w = static_cast<const int8_t*>(d.w);
    b.n = d.n;
    b.ih = d.ih;
    b.iw = d.iw;
    b.ic = 2 * d.ic;
    b.oc = d.oc;
    b.kh = d.kh;
    b.kw = d.kw;
    b.oh = d.oh;
    b.ow = d.ow;
    b.pt = d.pt;
    b.pl = d.pl;
    b.dy = d.dy;
    b.dx = d.dx;
    b.wpack = static_cast<const int8_t*>(d.wpack);
    return b;
}

bool f16_halo_ok(const ConvF16Desc& d)
{
    const bool aligned = (reinterpret_cast<uintptr_t>(d.x) | reinterpret_cast<uintptr_t>(d.w)) % 16 == 0;
    return aligned && d.sy == 1 && d.sx == 1 && d.ic % 16 == 0 && (d.elem == ELEM_BF16 || d.elem == ELEM_F16) &&
           (d.out_fmt == FMT_F32 || d.out_fmt == FMT_BF16 || d.out_fmt == FMT_F16) &&
           int64_t(d.n) * d.ih * d.iw * d.ic * 2 < (int64_t(1) << 31) &&
           int64_t(d.n) * d.oh * d.ow * d.oc * 4 < (int64_t(1) << 31);
}

// Zeros for the padding taps of float halo convolutions (the int8 kind
// loads the input zero point from its table instead); one address per
// device, as hipGetSymbolAddress reports it.
__device__ __attribute__((aligned(16))) int32_t h32_float_zeros[4];

const int8_t* float_zeros()
{
    static const int8_t* addr[64] = {nullptr};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= 64)
        throw std::runtime_error("conv_f16_halo: device index out of range");
    if (!addr[dev]) {
        void* p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(h32_float_zeros)), "halo zero fill");
        addr[dev] = static_cast<const int8_t*>(p);
    }
    return addr[dev];
}

template <int BC, int PG, int TB, int KT, int EL>
void launch_halo32_float(const Halo32Args& a, unsigned blocks, size_t lds, FloatFmt fmt, hipStream_t s)
{
    if (fmt == FMT_F32)
        launch_halo32<BC, PG, TB, KT, 4, false, false, EL>(a, blocks, lds, s);
    else
        launch_halo32<BC, PG, TB, KT, 2, false, false, EL>(a, blocks, lds, s);
}

template <int EL>
void launch_halo32_float_layout(const Halo32Args& a, int bc, unsigned blocks, size_t lds, bool k3, FloatFmt fmt,
                                hipStream_t s)
{
    if (bc == 128) {
        if (k3)
            launch_halo32_float<128, 4, 2, 9, EL>(a, blocks, lds, fmt, s);
        else
            launch_halo32_float<128, 4, 2, 0, EL>(a, blocks, lds, fmt, s);
    } else if (a.TB == 2) {
        if (k3)
            launch_halo32_float<64, 8, 2, 9, EL>(a, blocks, lds, fmt, s);
        else
            launch_halo32_float<64, 8, 2, 0, EL>(a, blocks, lds, fmt, s);
    } else {
        if (k3)
            launch_halo32_float<64, 8, 1, 9, EL>(a, blocks, lds, fmt, s);
        else
            launch_halo32_float<64, 8, 1, 0, EL>(a, blocks, lds, fmt, s);
    }
}

}  // namespace

int conv_f16_halo_block(const ConvF16Desc& d)
{
    if (!f16_halo_ok(d))
        return 0;
    const ConvI8Desc b = f16_byte_desc(d);
    Halo32Args a{};
    int bc = 0;
    size_t lds = 0;
    unsigned blocks = 0;
    return halo32_plan(b, false, a, bc, lds, blocks, false) ? bc : 0;
}

int64_t conv_f16_halo_wpack_bytes(const ConvF16Desc& d)
{
    const int bc = conv_f16_halo_block(d);
    if (bc == 0)
        return 0;
    return int64_t((d.oc + bc - 1) / bc) * bc * d.kh * d.kw * 2 * d.ic;
}

void conv_f16_halo_wpack(const ConvF16Desc& d, void* wp, hipStream_t stream)
{
    const ConvI8Desc b = f16_byte_desc(d);
    Halo32Args a{};
    int bc = 0;
    size_t lds = 0;
    unsigned blocks = 0;
    if (!f16_halo_ok(d) || !halo32_plan(b, false, a, bc, lds, blocks, false))
        throw std::runtime_error("conv_f16_halo_wpack: the halo kernel does not apply");
    const int64_t slots = int64_t((d.oc + bc - 1) / bc) * bc * d.kh * d.kw * b.ic / 16;
    hipLaunchKernelGGL(conv_i8_wpack_kernel, dim3(unsigned((slots + 255) / 256)), dim3(256), 0, stream, b.w, d.oc,
                       d.kh * d.kw * b.ic, b.ic, d.kh * d.kw, bc, slots, static_cast<v4u*>(wp));
}

void conv_f16_halo(const ConvF16Desc& d, void* out, hipStream_t stream)
{
    const ConvI8Desc b = f16_byte_desc(d);
    Halo32Args a{};
    int bc = 0;
    size_t lds = 0;
    unsigned blocks = 0;
    if (!f16_halo_ok(d) || !d.wpack || !halo32_plan(b, false, a, bc, lds, blocks, false))
        throw std::runtime_error("conv_f16_halo: the halo kernel does not apply");
    if (int64_t(d.n) * d.oh * d.ow <= 0 || d.oc <= 0)
        return;
    a.tab = nullptr;
    a.zfill = float_zeros();
    a.E = EpiArgs{};
    a.E.out = static_cast<uint8_t*>(out);
    a.E.N = d.oc;
    a.fbias = d.bias;
    a.fbias_len = d.bias_len;
    a.fmt = d.out_fmt;
    const bool k3 = d.kh == 3 && d.kw == 3;
    if (d.elem == ELEM_BF16)
        launch_halo32_float_layout<HE_BF16>(a, bc, blocks, lds, k3, d.out_fmt, stream);
    else
        launch_halo32_float_layout<HE_F16>(a, bc, blocks, lds, k3, d.out_fmt, stream);
}

}  // namespace kern
}  // namespace tosa
