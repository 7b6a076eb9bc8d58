// Implicit-GEMM CONV2D and batched MATMUL on CDNA4 MFMA.
//
// Replaces the reference's scalar loops ConvNd::accumulate
// (src/ops/conv.rs:149-181) and Dims::run (src/ops/matmul.rs:80-95) for the
// hot types: int8 x int8/int4 with int32 accumulation
// (v_mfma_i32_16x16x64_i8) and bf16/fp16 with fp32 accumulation
// (v_mfma_f32_16x16x32_{bf16,f16}).
//
// GEMM view: D[c][p] = sum_k Q[c][k] * P[p][k], where p runs over output
// pixels (conv: n*oh*ow; matmul: h) and c over output channels (conv: oc;
// matmul: w). The channel side is the MFMA "A" operand, so each lane ends up
// holding consecutive output channels of one pixel and the NHWC store is a
// contiguous vector store.
//
// Zero points are folded rather than subtracted, because x - zp spans 9 bits
// and no longer fits int8 MFMA operands:
//   sum_k (x - zx)(w - zw) = sum x w - zw sum x - zx sum w + K zx zw  (mod 2^32)
// Padding taps are loaded as zx so that their (x - zx) term vanishes, which is
// the reference's "skip taps outside the input" (src/ops/conv.rs:162-167).
//
// Tiles: BM channels x BN pixels per 256-thread workgroup (4 waves), K staged
// 64 bytes at a time through double-buffered LDS (rows padded to 80 bytes so
// the 16-byte fragment reads of a wave hit distinct banks).
#include <type_traits>

#include "kcommon.h"

namespace tosa {
namespace kern {

FastDiv::FastDiv(uint32_t div) : d(div)
{
    uint32_t sh = 0;
    while ((uint64_t(1) << sh) < div)
        sh++;
    s = sh;
    m = static_cast<uint32_t>(((uint64_t(1) << 32) * ((uint64_t(1) << sh) - div)) / div + 1);
}

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int LDS_ROW = 80;  // 64 data bytes + 16 pad

struct GemmArgs {
    const uint8_t* P;  // pixel side: conv input / matmul A
    const uint8_t* Q;  // channel side: conv weight / matmul B
    uint8_t* out;
    int32_t M, N, K;  // pixels, channels, reduction length (elements)
    // conv geometry
    int32_t ih, iw, ic, kw, ohow, ow, pt, pl, sy, sx, dy, dx;
    FastDiv div_ic, div_kw, div_ohow, div_ow;
    // matmul batch strides (elements)
    int64_t p_bstride, q_bstride, o_bstride;
    int32_t zp_x, zp_w;
    const int32_t* wsum;
    const void* bias;
    int32_t bias_len;
    int32_t epi;
    RescaleDev rs;
    int32_t out_fmt;
    uint32_t* err;
};

template <int VEC>
struct VecT;
template <>
struct VecT<16> {
    using T = uint4;
};
template <>
struct VecT<8> {
    using T = uint2;
};
template <>
struct VecT<4> {
    using T = uint32_t;
};
template <>
struct VecT<2> {
    using T = uint16_t;
};
template <>
struct VecT<1> {
    using T = uint8_t;
};

template <int VEC>
__device__ __forceinline__ void copy_vec(uint8_t* dst, const uint8_t* src)
{
    using T = typename VecT<VEC>::T;
    *reinterpret_cast<T*>(dst) = *reinterpret_cast<const T*>(src);
}

template <int VEC>
__device__ __forceinline__ void fill_vec(uint8_t* dst, uint32_t word)
{
#pragma unroll
    for (int i = 0; i < VEC; i++)
        dst[i] = static_cast<uint8_t>(word >> (8 * (i & 3)));
}

template <int ES>
__device__ __forceinline__ v4f mfma_f(const v4i& a, const v4i& b, const v4f& c, int elem)
{
    if (elem == ELEM_BF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0,
                                                       0);
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}

// ES: element bytes (1: int8, 2: bf16/f16). VEC: bytes per global load on
// the pixel side (and the conv weight side). CONV: implicit conv vs matmul.
template <int ES, int BM, int BN, int WM, int WN, int VEC, bool CONV>
__global__ void __launch_bounds__(256) igemm_kernel(GemmArgs A, int elem)
{
    constexpr bool INT = (ES == 1);
    constexpr int TM = BM / WM / 16;
    constexpr int TN = BN / WN / 16;
    constexpr int PB = BN / 64;                         // pixel rows per thread
    constexpr int QCH = (BM * 4 + 255) / 256;           // conv weight chunks per thread
    constexpr int KE = 64 / ES;                         // elements per K step
    constexpr int QT = (ES == 1) ? (BM * 4 + 255) / 256 : (BM * 8 + 255) / 256;  // matmul transpose blocks
    static_assert(TM >= 1 && TN >= 1 && WM * WN == 4, "tile");

    __shared__ __attribute__((aligned(16))) uint8_t sQ[2][BM * LDS_ROW];
    __shared__ __attribute__((aligned(16))) uint8_t sP[2][BN * LDS_ROW];
    __shared__ int32_t s_rowsum[BN];
    __shared__ int32_t s_colsum[BM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int wave_c0 = wm * (BM / WM);
    const int wave_p0 = wn * (BN / WN);
    const int m0 = blockIdx.x * BN;
    const int n0 = blockIdx.y * BM;
    const int bz = blockIdx.z;

    const uint8_t* P = A.P + (CONV ? 0 : int64_t(bz) * A.p_bstride * ES);
    const uint8_t* Q = A.Q + (CONV ? 0 : int64_t(bz) * A.q_bstride * ES);

    const bool need_rowsum = INT && A.zp_w != 0;
    const bool need_colsum = INT && !CONV && A.zp_x != 0;
    if (need_rowsum)
        for (int i = tid; i < BN; i += 256)
            s_rowsum[i] = 0;
    if (need_colsum)
        for (int i = tid; i < BM; i += 256)
            s_colsum[i] = 0;

    // ---- pixel-side rows owned by this thread -----------------------------
    const int pcol = tid & 3;  // 16-byte segment of the 64-byte K step
    int32_t p_iy0[PB], p_ix0[PB];
    int64_t p_base[PB];
    bool p_ok[PB];
#pragma unroll
    for (int p = 0; p < PB; p++) {
        const int row = (tid >> 2) + 64 * p;
        const int m = m0 + row;
        p_ok[p] = m < A.M;
        const int mm = p_ok[p] ? m : 0;
        if constexpr (CONV) {
            const int b = fdiv(mm, A.div_ohow);
            const int rem = mm - b * A.ohow;
            const int oy = fdiv(rem, A.div_ow);
            const int ox = rem - oy * A.ow;
            p_iy0[p] = oy * A.sy - A.pt;
            p_ix0[p] = ox * A.sx - A.pl;
            p_base[p] = int64_t(b) * A.ih * A.iw * A.ic;
        } else {
            p_iy0[p] = 0;
            p_ix0[p] = 0;
            p_base[p] = int64_t(mm) * A.K;
        }
    }
    const uint32_t zfill = INT ? (uint32_t(uint8_t(A.zp_x)) * 0x01010101u) : 0u;
    int32_t rsum[PB];
#pragma unroll
    for (int p = 0; p < PB; p++)
        rsum[p] = 0;
    int32_t csum[4] = {0, 0, 0, 0};

    uint4 preg[PB];
    uint4 qreg[QCH];
    uint32_t treg[QT][4 / ES];  // matmul: transposed words

    const int nsteps = (A.K + KE - 1) / KE;

    auto load_p = [&](int step) {
        const int kel0 = step * KE;
#pragma unroll
        for (int p = 0; p < PB; p++) {
            uint8_t* dst = reinterpret_cast<uint8_t*>(&preg[p]);
#pragma unroll
            for (int j = 0; j < 16 / VEC; j++) {
                const int k = kel0 + (pcol * 16 + j * VEC) / ES;
                if (k < A.K && p_ok[p]) {
                    if constexpr (CONV) {
                        const int tap = fdiv(k, A.div_ic);
                        const int cc = k - tap * A.ic;
                        const int ky = fdiv(tap, A.div_kw);
                        const int kx = tap - ky * A.kw;
                        const int iy = p_iy0[p] + ky * A.dy;
                        const int ix = p_ix0[p] + kx * A.dx;
                        if (unsigned(iy) < unsigned(A.ih) && unsigned(ix) < unsigned(A.iw))
                            copy_vec<VEC>(dst + j * VEC, P + (p_base[p] + (int64_t(iy) * A.iw + ix) * A.ic + cc) * ES);
                        else
                            fill_vec<VEC>(dst + j * VEC, zfill);
                    } else {
                        copy_vec<VEC>(dst + j * VEC, P + (p_base[p] + k) * ES);
                    }
                } else {
                    fill_vec<VEC>(dst + j * VEC, 0u);
                }
            }
            if (need_rowsum) {
                const uint32_t* w = reinterpret_cast<const uint32_t*>(&preg[p]);
                int32_t s = rsum[p];
#pragma unroll
                for (int q = 0; q < 4; q++)
                    s = __builtin_amdgcn_sdot4(static_cast<int>(w[q]), 0x01010101, s, false);
                rsum[p] = s;
            }
        }
    };

    auto load_q = [&](int step) {
        const int kel0 = step * KE;
        if constexpr (CONV) {
#pragma unroll
            for (int i = 0; i < QCH; i++) {
                const int q = tid + 256 * i;
                uint8_t* dst = reinterpret_cast<uint8_t*>(&qreg[i]);
                const int row = q >> 2, col = q & 3;
                const int oc = n0 + row;
#pragma unroll
                for (int j = 0; j < 16 / VEC; j++) {
                    const int k = kel0 + (col * 16 + j * VEC) / ES;
                    if (q < BM * 4 && oc < A.N && k < A.K)
                        copy_vec<VEC>(dst + j * VEC, Q + (int64_t(oc) * A.K + k) * ES);
                    else
                        fill_vec<VEC>(dst + j * VEC, 0u);
                }
            }
        } else {
            // B is [K][N] (row-major, N contiguous): load (4/ES) x (4/ES)
            // element blocks and transpose them so LDS holds B^T rows.
            constexpr int EPW = 4 / ES;        // elements per 32-bit word
            constexpr int WB = BM / EPW;       // word-blocks across the channel tile
#pragma unroll
            for (int i = 0; i < QT; i++) {
                const int q = tid + 256 * i;
                const int wb = q % WB, kb = q / WB;
                const int n = n0 + wb * EPW;
                const int k = kel0 + kb * EPW;
                uint32_t rows[EPW];
#pragma unroll
                for (int r = 0; r < EPW; r++) {
                    uint32_t word = 0;
                    if (q < WB * 16 && k + r < A.K) {
                        const uint8_t* src = Q + (int64_t(k + r) * A.N + n) * ES;
                        if (n + EPW <= A.N && ((A.N * ES) & 3) == 0) {
                            word = *reinterpret_cast<const uint32_t*>(src);
                        } else {
#pragma unroll
                            for (int e = 0; e < EPW; e++)
                                if (n + e < A.N) {
                                    uint32_t v = ES == 1 ? uint32_t(src[e])
                                                         : uint32_t(*reinterpret_cast<const uint16_t*>(src + 2 * e));
                                    word |= v << (8 * ES * e);
                                }
                        }
                    }
                    rows[r] = word;
                }
#pragma unroll
                for (int e = 0; e < EPW; e++) {
                    uint32_t t = 0;
#pragma unroll
                    for (int r = 0; r < EPW; r++) {
                        const uint32_t v = (rows[r] >> (8 * ES * e)) & (ES == 1 ? 0xFFu : 0xFFFFu);
                        t |= v << (8 * ES * r);
                    }
                    treg[i][e] = t;
                    if (need_colsum)
                        csum[e] = __builtin_amdgcn_sdot4(static_cast<int>(t), 0x01010101, csum[e], false);
                }
            }
        }
    };

    auto store_lds = [&](int buf) {
#pragma unroll
        for (int p = 0; p < PB; p++) {
            const int row = (tid >> 2) + 64 * p;
            *reinterpret_cast<uint4*>(&sP[buf][row * LDS_ROW + pcol * 16]) = preg[p];
        }
        if constexpr (CONV) {
#pragma unroll
            for (int i = 0; i < QCH; i++) {
                const int q = tid + 256 * i;
                if (q < BM * 4)
                    *reinterpret_cast<uint4*>(&sQ[buf][(q >> 2) * LDS_ROW + (q & 3) * 16]) = qreg[i];
            }
        } else {
            constexpr int EPW = 4 / ES;
            constexpr int WB = BM / EPW;
#pragma unroll
            for (int i = 0; i < QT; i++) {
                const int q = tid + 256 * i;
                if (q < WB * 16) {
                    const int wb = q % WB, kb = q / WB;
#pragma unroll
                    for (int e = 0; e < EPW; e++)
                        *reinterpret_cast<uint32_t*>(&sQ[buf][(wb * EPW + e) * LDS_ROW + kb * 4]) = treg[i][e];
                }
            }
        }
    };

    using AccV = typename std::conditional<INT, v4i, v4f>::type;
    AccV acc[TM][TN];
#pragma unroll
    for (int a = 0; a < TM; a++)
#pragma unroll
        for (int b = 0; b < TN; b++)
            acc[a][b] = AccV{0, 0, 0, 0};

    load_p(0);
    load_q(0);
    store_lds(0);
    __syncthreads();

    const int frag_k = (lane >> 4) * 16;
    const int r16 = lane & 15;
    for (int step = 0; step < nsteps; step++) {
        const int buf = step & 1;
        if (step + 1 < nsteps) {
            load_p(step + 1);
            load_q(step + 1);
        }
        v4i af[TM], bf[TN];
#pragma unroll
        for (int tm = 0; tm < TM; tm++) {
            const int row = wave_c0 + (r16 >> 2) * (4 * TM) + 4 * tm + (r16 & 3);
            af[tm] = *reinterpret_cast<const v4i*>(&sQ[buf][row * LDS_ROW + frag_k]);
        }
#pragma unroll
        for (int tn = 0; tn < TN; tn++) {
            const int row = wave_p0 + 16 * tn + r16;
            bf[tn] = *reinterpret_cast<const v4i*>(&sP[buf][row * LDS_ROW + frag_k]);
        }
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int tn = 0; tn < TN; tn++) {
                if constexpr (INT)
                    acc[tm][tn] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[tm], bf[tn], acc[tm][tn], 0, 0, 0);
                else
                    acc[tm][tn] = mfma_f<ES>(af[tm], bf[tn], acc[tm][tn], elem);
            }
        if (step + 1 < nsteps)
            store_lds(buf ^ 1);
        __syncthreads();
    }

    // ---- zero-point sums -------------------------------------------------
    if (INT && need_rowsum) {
#pragma unroll
        for (int p = 0; p < PB; p++) {
            int32_t s = rsum[p];
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            if (pcol == 0)
                s_rowsum[(tid >> 2) + 64 * p] = s;
        }
    }
    if (INT && need_colsum) {
        constexpr int EPW = 4;
        constexpr int WB = BM / EPW;
        if (tid < WB * 16) {  // the same word-block in every K step (256 % WB == 0)
            const int wb = tid % WB;
#pragma unroll
            for (int e = 0; e < EPW; e++)
                atomicAdd(&s_colsum[wb * EPW + e], csum[e]);
        }
    }
    if (INT && (need_rowsum || need_colsum))
        __syncthreads();

    // ---- epilogue --------------------------------------------------------
    uint32_t err = 0;
    const int ob = A.epi == EPI_FLOAT ? (A.out_fmt == FMT_F32 ? 4 : 2) : (A.epi == EPI_I32 ? 4 : A.rs.out_bytes);
    const int cb = wave_c0 + (lane >> 4) * (4 * TM);  // first channel (tile-relative)
    const uint32_t kzz = uint32_t(A.K) * uint32_t(A.zp_x) * uint32_t(A.zp_w);
#pragma unroll
    for (int tn = 0; tn < TN; tn++) {
        const int pl = wave_p0 + 16 * tn + r16;
        const int m = m0 + pl;
        if (m >= A.M)
            continue;
        const int32_t rs_pix = (INT && need_rowsum) ? s_rowsum[pl] : 0;
        const int64_t orow = CONV ? int64_t(m) * A.N : int64_t(bz) * A.o_bstride + int64_t(m) * A.N;
        uint32_t vals[TM * 4];
#pragma unroll
        for (int tm = 0; tm < TM; tm++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int cl = cb + 4 * tm + i;
                const int c = n0 + cl;
                const int cc = c < A.N ? c : A.N - 1;
                uint32_t v;
                if constexpr (INT) {
                    uint32_t a = uint32_t(acc[tm][tn][i]);
                    a -= uint32_t(A.zp_w) * uint32_t(rs_pix);
                    if (A.zp_x != 0) {
                        const int32_t ws = CONV ? A.wsum[cc] : s_colsum[cl];
                        a -= uint32_t(A.zp_x) * uint32_t(ws);
                    }
                    a += kzz;
                    if (CONV && A.bias)
                        a += uint32_t(static_cast<const int32_t*>(A.bias)[A.bias_len == 1 ? 0 : cc]);
                    if (A.epi == EPI_RESCALE) {
                        const int ch = A.rs.per_channel ? cc : 0;
                        v = uint32_t(rescale_value(int64_t(int32_t(a)), A.rs.mult[ch], A.rs.shift[ch], A.rs, err));
                    } else {
                        v = a;
                    }
                } else {
#pragma clang fp contract(off)
                    const float accv = acc[tm][tn][i];
                    const float bv =
                        (CONV && A.bias) ? static_cast<const float*>(A.bias)[A.bias_len == 1 ? 0 : cc] : 0.0f;
                    float r = (CONV && A.bias) ? round_fmt16(round_fmt16(accv, A.out_fmt) + bv, A.out_fmt) : accv;
                    v = A.out_fmt == FMT_F32 ? __builtin_bit_cast(uint32_t, r)
                                             : uint32_t(A.out_fmt == FMT_F16 ? f32_to_f16_bits(r) : f32_to_bf16_bits(r));
                }
                vals[tm * 4 + i] = v;
            }
        const int c0 = n0 + cb;
        uint8_t* dst = A.out + (orow + c0) * ob;
        const bool full = c0 + 4 * TM <= A.N;
        if (ob == 1 && full && (((orow + c0) & 3) == 0)) {
#pragma unroll
            for (int w = 0; w < TM; w++) {
                const uint32_t word = (vals[4 * w] & 0xFF) | ((vals[4 * w + 1] & 0xFF) << 8) |
                                      ((vals[4 * w + 2] & 0xFF) << 16) | ((vals[4 * w + 3] & 0xFF) << 24);
                *reinterpret_cast<uint32_t*>(dst + 4 * w) = word;
            }
        } else if (ob == 2 && full && (((orow + c0) & 1) == 0)) {
#pragma unroll
            for (int w = 0; w < 2 * TM; w++)
                *reinterpret_cast<uint32_t*>(dst + 4 * w) = (vals[2 * w] & 0xFFFF) | (vals[2 * w + 1] << 16);
        } else if (ob == 4 && full && (((orow + c0) & 3) == 0)) {
#pragma unroll
            for (int w = 0; w < TM; w++)
                *reinterpret_cast<uint4*>(dst + 16 * w) =
                    uint4{vals[4 * w], vals[4 * w + 1], vals[4 * w + 2], vals[4 * w + 3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4 * TM; e++) {
                if (c0 + e >= A.N)
                    continue;
                if (ob == 1)
                    dst[e] = uint8_t(vals[e]);
                else if (ob == 2)
                    reinterpret_cast<uint16_t*>(dst)[e] = uint16_t(vals[e]);
                else
                    reinterpret_cast<uint32_t*>(dst)[e] = vals[e];
            }
        }
    }
    report(A.err, err);
}

template <int ES, int BM, int BN, int WM, int WN, int VEC, bool CONV>
void launch_tile(const GemmArgs& a, int elem, int batch, hipStream_t s)
{
    dim3 grid((a.M + BN - 1) / BN, (a.N + BM - 1) / BM, batch);
    hipLaunchKernelGGL((igemm_kernel<ES, BM, BN, WM, WN, VEC, CONV>), grid, dim3(256), 0, s, a, elem);
}

template <int ES, int VEC, bool CONV>
void launch_vec(const GemmArgs& a, int elem, int batch, hipStream_t s)
{
    if (a.N > 64)
        launch_tile<ES, 128, 128, 2, 2, VEC, CONV>(a, elem, batch, s);
    else if (a.N > 32)
        launch_tile<ES, 64, 128, 1, 4, VEC, CONV>(a, elem, batch, s);
    else if (a.N > 16)
        launch_tile<ES, 32, 256, 1, 4, VEC, CONV>(a, elem, batch, s);
    else
        launch_tile<ES, 16, 256, 1, 4, VEC, CONV>(a, elem, batch, s);
}

template <int ES, bool CONV>
void launch_es(const GemmArgs& a, int elem, int batch, int align_elems, hipStream_t s)
{
    const int ab = align_elems * ES;  // bytes each pixel-side load may cover
    if (ab % 16 == 0)
        launch_vec<ES, 16, CONV>(a, elem, batch, s);
    else if (ab % 8 == 0)
        launch_vec<ES, 8, CONV>(a, elem, batch, s);
    else if (ab % 4 == 0)
        launch_vec<ES, 4, CONV>(a, elem, batch, s);
    else if (ab % 2 == 0)
        launch_vec<ES, 2, CONV>(a, elem, batch, s);
    else
        launch_vec<ES, 1, CONV>(a, elem, batch, s);
}

}  // namespace

void gemm(const GemmDesc& d, const void* x, const void* w, void* out, uint32_t* err, hipStream_t stream)
{
    GemmArgs a{};
    a.P = static_cast<const uint8_t*>(x);
    a.Q = static_cast<const uint8_t*>(w);
    a.out = static_cast<uint8_t*>(out);
    a.zp_x = d.zp_x;
    a.zp_w = d.zp_w;
    a.wsum = d.wsum;
    a.bias = d.bias;
    a.bias_len = d.bias_len;
    a.epi = d.epi;
    a.rs = d.rs;
    a.out_fmt = d.out_fmt;
    a.err = err;
    int batch = 1, align;
    if (d.is_conv) {
        a.M = d.n * d.oh * d.ow;
        a.N = d.oc;
        a.K = d.kh * d.kw * d.ic;
        a.ih = d.ih;
        a.iw = d.iw;
        a.ic = d.ic;
        a.kw = d.kw;
        a.ohow = d.oh * d.ow;
        a.ow = d.ow;
        a.pt = d.pt;
        a.pl = d.pl;
        a.sy = d.sy;
        a.sx = d.sx;
        a.dy = d.dy;
        a.dx = d.dx;
        a.div_ic = FastDiv(d.ic);
        a.div_kw = FastDiv(d.kw);
        a.div_ohow = FastDiv(a.ohow);
        a.div_ow = FastDiv(d.ow);
        align = d.ic;  // a pixel-side load stays inside one tap; K % ic == 0
    } else {
        a.M = d.h;
        a.N = d.w;
        a.K = d.c;
        a.p_bstride = int64_t(d.h) * d.c;
        a.q_bstride = int64_t(d.c) * d.w;
        a.o_bstride = int64_t(d.h) * d.w;
        batch = d.batch;
        align = d.c;  // a row of A is c contiguous elements
    }
    // Power-of-two part of the alignment, so loads never straddle a row/tap.
    int al = 1;
    while (al < 16 && align % (2 * al) == 0)
        al *= 2;
    if (d.elem == ELEM_I8) {
        if (d.is_conv)
            launch_es<1, true>(a, d.elem, batch, al, stream);
        else
            launch_es<1, false>(a, d.elem, batch, al, stream);
    } else {
        if (d.is_conv)
            launch_es<2, true>(a, d.elem, batch, al, stream);
        else
            launch_es<2, false>(a, d.elem, batch, al, stream);
    }
}

namespace {
__global__ void weight_sums_kernel(const int8_t* w, int32_t oc, int32_t k, int32_t* wsum)
{
    const int o = blockIdx.x;
    int32_t s = 0;
    for (int i = threadIdx.x; i < k; i += blockDim.x)
        s += w[int64_t(o) * k + i];
    for (int off = 32; off > 0; off >>= 1)
        s += __shfl_down(s, off);
    __shared__ int32_t part[4];
    if ((threadIdx.x & 63) == 0)
        part[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0)
        wsum[o] = part[0] + part[1] + part[2] + part[3];
}
}  // namespace

void weight_sums_i8(const int8_t* w, int32_t oc, int32_t k, int32_t* wsum, hipStream_t stream)
{
    if (oc > 0)
        hipLaunchKernelGGL(weight_sums_kernel, dim3(oc), dim3(256), 0, stream, w, oc, k, wsum);
}

}  // namespace kern
}  // namespace tosa
