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
    int32_t out_zp;          // RESCALE output zero point, |out_zp| < 2^30
    int32_t clo, chi;        // output type range, narrowed to the CLAMP bounds if fused
    uint32_t* err;
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
template <int TM, int TN, int OB, bool RS, bool ZW, typename PixelMap>
__device__ __forceinline__ void epilogue(v4i (&acc)[TM][TN], const v4i* s_tab, const int32_t* s_rowsum, int cl0,
                                         int n0, int wave_p0, int j16, const EpiArgs& E, PixelMap pixel)
{
    constexpr int WORDS = TM * OB;  // 32-bit words of output per lane and pixel
    const int c0 = n0 + cl0;
    uint32_t res[TN][WORDS];
    bool bad_range = false;
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
                zwx = int32_t(uint32_t(E.zp_w) * uint32_t(s_rowsum[wave_p0 + 16 * tn + j16]));
            int32_t v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int32_t x = int32_t(uint32_t(acc[tm][tn][i]) + uint32_t(t0[i].x) - uint32_t(zwx));
                if constexpr (RS) {
                    // apply_scale_32: the value must lie in [-2^(s-1), 2^(s-1)),
                    // a condition on int32 values only for shifts below 32
                    // (t0.z = min(s - 1, 31)).
                    bad_range |= uint32_t((x >> t0[i].z) + 1) > 1u;
                    const int64_t rp = __builtin_bit_cast(int64_t, v2i{t1[i].x, t1[i].y});
                    const int64_t rn = __builtin_bit_cast(int64_t, v2i{t1[i].z, t1[i].w});
                    // With the value in range and 0 <= multiplier < 2^31 the
                    // scaled result always fits int32 (|r| <= 2^30 + 1), so
                    // apply_scale_32's result REQUIRE cannot fail, and with
                    // |output zp| < 2^30 neither can RESCALE's int32 check.
                    const int32_t r = int32_t((int64_t(x) * int64_t(t0[i].y) + (x >= 0 ? rp : rn)) >> t0[i].w);
                    // Output range and CLAMP in one step: the CLAMP bounds lie
                    // inside the output type's range, so clamping to the
                    // type and then to [clo, chi] is clamping to [clo, chi].
                    v[i] = med3(r + E.out_zp, E.clo, E.chi);
                } else {
                    v[i] = x;
                }
            }
            if constexpr (OB == 1) {
                res[tn][tm] = (uint32_t(v[0]) & 0xFF) | ((uint32_t(v[1]) & 0xFF) << 8) |
                              ((uint32_t(v[2]) & 0xFF) << 16) | (uint32_t(v[3]) << 24);
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
        }
    }

#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int m = pixel(wave_p0 + 16 * tn + j16);
        if (m < 0)
            continue;
        const int64_t o = int64_t(m) * E.N + c0;
        uint8_t* dst = E.out + o * OB;
        constexpr int VB = 4 * WORDS;  // bytes this lane holds for the pixel
        if (c0 + 4 * TM <= E.N && ((o * OB) % (VB < 16 ? VB : 16)) == 0) {
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
    if (bad_range)
        atomicOr(E.err, DERR_SCALE_RANGE);
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
    epilogue<TM, TN, OB, RS, ZW>(acc, s_tab, s_rowsum, wave_c0 + grp * 4 * TM, n0, wave_p0, j16, A.E,
                                 [&](int p) { return m0 + p < A.M ? m0 + p : -1; });
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
    epilogue<TM, TN, OB, RS, ZW>(acc, s_tab, s_rowsum, wave_c0 + grp * 4 * TM, n0, wave_p0, j16, A.E,
                                 [&](int p) { return p < npix ? m0 + p : -1; });
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
    constexpr int TN = 4;  // 16-pixel tiles per workgroup
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j16 = lane & 15;
    const int grp = lane >> 4;
    const int p0 = blockIdx.x * (16 * TN);
    const uint32_t zf = uint32_t(uint8_t(A.zp_x)) * 0x01010101u;
    const v4u zfill = v4u{zf, zf, zf, zf};

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

    const int cg = blockIdx.y * 4 + wave;
    if (cg < (A.C >> 4)) {
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
        bool bad_range = false;
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            v4i acc = v4i{0, 0, 0, 0}, acc1 = v4i{0, 0, 0, 0};
#pragma unroll
            for (int g = 0; g < G; g++) {
                const int iy = iy0[tn] + tdy[g];
                const int ix = ix0[tn] + tdx[g];
                const bool ok = tok[g] && unsigned(iy) < unsigned(A.IH) && unsigned(ix) < unsigned(A.IW);
                const v4u v = ld16(A.x + (ok ? (pbase[tn] + iy * A.IW + ix) * A.C + c0 : 0));
                const v4i bx = __builtin_bit_cast(v4i, ok ? v : zfill);
                acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[g], bx, acc, 0, 0, 0);
                if constexpr (ZW)
                    acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wo[g], bx, acc1, 0, 0, 0);
            }
            if (!pok[tn])
                continue;
            int32_t v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int32_t xv = int32_t(uint32_t(acc[i]) + uint32_t(t0[i].x));
                if constexpr (ZW)
                    xv = int32_t(uint32_t(xv) - uint32_t(A.E.zp_w) * uint32_t(acc1[i]));
                if constexpr (RS) {
                    bad_range |= uint32_t((xv >> t0[i].z) + 1) > 1u;
                    const int64_t rp = __builtin_bit_cast(int64_t, v2i{t1[i].x, t1[i].y});
                    const int64_t rn = __builtin_bit_cast(int64_t, v2i{t1[i].z, t1[i].w});
                    const int32_t r = int32_t((int64_t(xv) * int64_t(t0[i].y) + (xv >= 0 ? rp : rn)) >> t0[i].w);
                    v[i] = med3(r + A.E.out_zp, A.E.clo, A.E.chi);
                } else {
                    v[i] = xv;
                }
            }
            uint8_t* dst = A.E.out + (int64_t(p0 + 16 * tn + j16) * A.C + c0 + 4 * grp) * OB;
            if constexpr (OB == 1)
                *reinterpret_cast<uint32_t*>(dst) = (uint32_t(v[0]) & 0xFF) | ((uint32_t(v[1]) & 0xFF) << 8) |
                                                    ((uint32_t(v[2]) & 0xFF) << 16) | (uint32_t(v[3]) << 24);
            else if constexpr (OB == 2)
                *reinterpret_cast<v2u*>(dst) = v2u{(uint32_t(v[0]) & 0xFFFF) | (uint32_t(v[1]) << 16),
                                                   (uint32_t(v[2]) & 0xFFFF) | (uint32_t(v[3]) << 16)};
            else
                *reinterpret_cast<v4i*>(dst) = v4i{v[0], v[1], v[2], v[3]};
        }
        if (bad_range)
            atomicOr(A.E.err, DERR_SCALE_RANGE);
    }
}

// One wave per output channel:
//   tab[2c]   = {bias + K zx zw - zx sum_k w[c][k] (mod 2^32), multiplier,
//                min(shift - 1, 31), shift}
//   tab[2c+1] = {rounding constant for values >= 0 (int64, lo/hi),
//                rounding constant for values < 0 (int64, lo/hi)}
// The rounding constants are apply_scale_32's 2^(s-1), plus or minus 2^30
// under double rounding for shifts above 31 (src/ops/quant.rs:26-29).
__global__ void conv_i8_table_kernel(const int8_t* w, int32_t N, int32_t K, int32_t cstride, int32_t kstride,
                                     const int32_t* bias, int32_t bias_len, int32_t zx, int32_t zw,
                                     const int32_t* mult, const int32_t* shift, int32_t per_channel, int32_t dbl,
                                     v4i* tab)
{
    const int c = blockIdx.x;
    const int lane = threadIdx.x;
    int32_t s = 0;
    if (zx != 0)
        for (int k = lane; k < K; k += 64)
            s += w[int64_t(c) * cstride + int64_t(k) * kstride];
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

template <int G, int OB, bool RS, bool ZW>
void launch_dw(const DwArgs& a, hipStream_t s)
{
    const unsigned blocks = unsigned((a.P + 63) / 64);
    hipLaunchKernelGGL((conv_i8_dw_kernel<G, OB, RS, ZW>), dim3(blocks, unsigned((a.C / 16 + 3) / 4)), dim3(256), 0, s,
                       a);
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
    hipLaunchKernelGGL(conv_i8_table_kernel, dim3(d.oc), dim3(64), 0, stream, d.w, d.oc, K, cstride, kstride, d.bias,
                       d.bias_len, d.zp_x, d.zp_w, rs ? rs->mult : nullptr, rs ? rs->shift : nullptr,
                       rs ? rs->per_channel : 0, rs ? int32_t(rs->rounding == 3) : 0, static_cast<v4i*>(tab));
}

bool conv_i8_fast_epilogue_ok(const RescaleDev& rs)
{
    // |out_zp| < 2^30 keeps r + out_zp inside int32 (|r| <= 2^30 + 1); every
    // legal zero point (int8, uint8, uint16, or 0 for int32) satisfies it.
    return rs.scale32 && (rs.rounding == 1 || rs.rounding == 3) && !rs.in_unsigned && rs.in_zp == 0 &&
           (rs.out_bytes == 1 || rs.out_bytes == 2 || rs.out_bytes == 4) && rs.out_zp > -(int64_t(1) << 30) &&
           rs.out_zp < (int64_t(1) << 30);
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
        e.out_zp = int32_t(rs->out_zp);
        // CLAMP bounds are values of the output type, so they lie inside
        // [lo, hi] (prepare_clamp_int decodes them in that type).
        e.clo = int32_t(rs->has_clamp ? std::max<int64_t>(rs->clamp_lo, rs->lo) : rs->lo);
        e.chi = int32_t(rs->has_clamp ? std::min<int64_t>(rs->clamp_hi, rs->hi) : rs->hi);
        ob = rs->out_bytes;
    }
    if (int64_t(d.n) * d.oh * d.ow <= 0 || d.oc <= 0)
        return;
    const bool zw = d.zp_w != 0;
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

    HaloArgs h{};
    int bc = 128, kc = 128;
    size_t lds = 0;
    unsigned blocks = 0;
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
