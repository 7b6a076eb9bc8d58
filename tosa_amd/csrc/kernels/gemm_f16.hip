// bf16 / fp16 GEMM with fp32 accumulation on v_mfma_f32_32x32x16_{bf16,f16}:
// batched MATMUL (A [b][M][K] x B [b][K][N]) and 1x1 stride-1 unpadded
// CONV2D (NHWC rows x OHWI rows) with the float epilogue.
//
// Replaces Dims::run (src/ops/matmul.rs:80-95) with AccF32
// (src/ops/accum.rs:59-71) for bf16/fp16 operands and fp32 output, and
// ConvNd::accumulate (src/ops/conv.rs:149-181) plus the float epilogue
// out = round(round(acc) + bias) (src/ops/conv.rs:493-495) for 1x1
// convolutions. The products are exact in fp32 and the sum is taken in a
// different order than the reference's sequential one, so results agree
// within the documented fp32 reassociation bound.
//
// C[m][n] = sum_k A[m][k] Bt[n][k]: the MFMA's A operand is a block of 32
// rows of A (pixels / matmul rows), its B operand 32 rows of Bt (output
// channels / matmul columns), so lane l's results are column n0 + l % 32 of
// rows 8 (i / 4) + 4 (l / 32) + i % 4: every store instruction writes two
// 128-byte row segments, and a conv bias is one value per lane.
//
// Workgroup tile 256 x 256, 8 waves of 128 (M) x 64 (N) (4 x 2 MFMA tiles,
// 6 fragment reads per 8 MFMAs), K staged 64 elements at a time through two
// LDS buffers. LDS image of one operand stage: the 16-byte chunk holding
// elements 16 j + 8 c .. + 7 of row r (block b = r / 32 of the tile) sits at
// slot ((8 j + b) 2 + c) 32 + ((r % 32) ^ b), so the fragment read of a row
// block (lane l: k-half l / 32) is one contiguous 1 KB, and lane l holds row
// 32 b + ((l % 32) ^ b); the epilogue undoes that permutation. The XOR keeps
// the 8-byte writes of the transposed B (eight row blocks at once) at two
// lanes per bank.
// A rows (and Bt rows when B is given transposed) arrive by direct
// global->LDS loads; a [K][N] B is loaded as 4 x 8 element blocks,
// transposed in registers with byte permutes, and written as 8-byte pieces
// of the rows of Bt.
#include "kcommon.h"

namespace tosa {
namespace kern {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lvoid;

constexpr int GT = 256;        // tile rows (M) and columns (N)
constexpr int GK = 64;         // K elements per stage
constexpr int GNT = 512;       // threads
constexpr int GSTAGE = GT * GK * 2;  // bytes of one operand stage (32 KB)

struct GemmF16Args {
    const uint16_t* a;   // [batch][M][K]
    const uint16_t* b;   // [batch][N][K] (NT) or [batch][K][N]
    uint8_t* out;        // [batch][M][N] of out_fmt
    const float* bias;   // per column (n), or null
    int32_t bias_len;
    int32_t M, N, K, batch;
    int32_t tiles_m, tiles_n;
    int64_t a_bs, b_bs, o_bs;  // batch strides (elements)
    int32_t out_fmt;
};

// A direct 16-byte global->LDS load (global_load_lds_dwordx4: lane l writes
// LDS byte address `l` + 16 l, `l` wave-uniform), issued through inline
// assembly so that the compiler's LDS wait counting leaves the fragment
// reads alone; the kernel waits for these loads itself (vmcnt(0) and a
// barrier) before reading what they fill.
__device__ __forceinline__ void dma16(const void* g, const void* l)
{
    const uint32_t la = __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>((const lvoid*)l)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(la) : "memory", "m0");
}

template <bool BF>
__device__ __forceinline__ v16f mfma32(const v4u& a, const v4u& b, const v16f& c)
{
    if constexpr (BF)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0,
                                                       0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0,
                                                      0);
}

// BF: bf16 (else fp16) operands. KN: B is [K][N] (else [N][K]).
template <bool BF, bool KN>
__global__ void __launch_bounds__(GNT, 2) gemm_f16_kernel(GemmF16Args A)
{
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* const sA = smem;                // [2][GSTAGE]
    uint8_t* const sB = smem + 2 * GSTAGE;   // [2][GSTAGE]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Workgroups go round-robin to the 8 XCDs; tile t of XCD x is workgroup
    // x + 8 t, so the tiles that run together on one XCD share A rows and Bt
    // rows in its L2.
    const int tiles = A.batch * A.tiles_m * A.tiles_n;
    const int tile = (tiles & 7) == 0 ? (blockIdx.x & 7) * (tiles >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int bz = tile / (A.tiles_m * A.tiles_n);
    const int rem = tile - bz * A.tiles_m * A.tiles_n;
    const int m0 = (rem / A.tiles_n) * GT;
    const int n0 = (rem - (rem / A.tiles_n) * A.tiles_n) * GT;
    const uint16_t* const ag = A.a + bz * A.a_bs;
    const uint16_t* const bg = A.b + bz * A.b_bs;

    // ---- staging ----------------------------------------------------------
    // DMA q fills slots 64 q .. + 63: k16 step j = q / 8, row block b = q % 8,
    // rows 32 b + ((l % 32) ^ b), k-half l / 32. Rows past the matrix re-read
    // its last row (their results are not stored).
    auto dma_rows = [&](const uint16_t* g, int rows, int r0, int k0, uint8_t* dst) {
        for (int q = wave; q < GSTAGE / 1024; q += GNT / 64) {
            const int j = q >> 3, row = 32 * (q & 7) + ((lane & 31) ^ (q & 7)), c = lane >> 5;
            const int r = r0 + row < rows ? r0 + row : rows - 1;
            dma16(g + int64_t(r) * A.K + k0 + 16 * j + 8 * c, dst + q * 1024);
        }
    };
    // [K][N] B: thread (nb, kq) loads rows k0 + 4 kq .. + 3, columns n0 + 8 nb
    // .. + 7 (columns past N read as zero).
    const int nb = tid & 31, kq = tid >> 5;
    v4u breg[4];
    auto load_kn = [&](int k0) {
        const int n = n0 + 8 * nb;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint16_t* src = bg + int64_t(k0 + 4 * kq + i) * A.N + (n < A.N ? n : 0);
            const v4u v = *reinterpret_cast<const v4u*>(src);
            breg[i] = n < A.N ? v : v4u{0, 0, 0, 0};
        }
    };
    auto store_kn = [&](uint8_t* dst) {
        // k = 4 kq + i lies in chunk (j, c) = (kq / 4, (kq % 4) / 2) at byte
        // 8 (kq % 2) + 2 i; column 8 nb + e is Bt row 8 nb + e.
        const int j = kq >> 2, c = (kq & 3) >> 1, off = 8 * (kq & 1);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
            const int d = e >> 1;
            const uint32_t lo = __builtin_amdgcn_perm(breg[1][d], breg[0][d], sel);
            const uint32_t hi = __builtin_amdgcn_perm(breg[3][d], breg[2][d], sel);
            const int row = 8 * nb + e;
            const int slot = ((8 * j + (row >> 5)) * 2 + c) * 32 + ((row & 31) ^ (row >> 5));
            *reinterpret_cast<v2u*>(dst + slot * 16 + off) = v2u{lo, hi};
        }
    };

    // ---- waves: 2 (M) x 4 (N), each 128 x 64 ------------------------------
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    v16f acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
            acc[a][b] = v16f{};

    const int nst = A.K / GK;
    dma_rows(ag, A.M, m0, 0, sA);
    if constexpr (KN) {
        load_kn(0);
        store_kn(sB);
    } else {
        dma_rows(bg, A.N, n0, 0, sB);
    }
    for (int st = 0; st < nst; st++) {
        const int buf = st & 1;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (st + 1 < nst) {
            dma_rows(ag, A.M, m0, (st + 1) * GK, sA + (buf ^ 1) * GSTAGE);
            if constexpr (KN)
                load_kn((st + 1) * GK);
            else
                dma_rows(bg, A.N, n0, (st + 1) * GK, sB + (buf ^ 1) * GSTAGE);
        }
        const uint8_t* const a_s = sA + buf * GSTAGE;
        const uint8_t* const b_s = sB + buf * GSTAGE;
        // Fragment of rows r0 .. r0 + 31 (r0 % 32 == 0) for k16 step j: one
        // contiguous 1 KB.
        auto frag = [&](const uint8_t* base, int j, int r0) {
            return *reinterpret_cast<const v4u*>(base + (8 * j + (r0 >> 5)) * 1024 + lane * 16);
        };
        v4u fa[2][4], fb[2][2];
#pragma unroll
        for (int a = 0; a < 4; a++)
            fa[0][a] = frag(a_s, 0, wm + 32 * a);
#pragma unroll
        for (int b = 0; b < 2; b++)
            fb[0][b] = frag(b_s, 0, wn + 32 * b);
#pragma unroll
        for (int j = 0; j < GK / 16; j++) {
            __builtin_amdgcn_sched_barrier(0);
            if (j + 1 < GK / 16) {
#pragma unroll
                for (int a = 0; a < 4; a++)
                    fa[(j + 1) & 1][a] = frag(a_s, j + 1, wm + 32 * a);
#pragma unroll
                for (int b = 0; b < 2; b++)
                    fb[(j + 1) & 1][b] = frag(b_s, j + 1, wn + 32 * b);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int a = 0; a < 4; a++)
                    acc[a][b] = mfma32<BF>(fa[j & 1][a], fb[j & 1][b], acc[a][b]);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (KN) {
            if (st + 1 < nst)
                store_kn(sB + (buf ^ 1) * GSTAGE);
        }
    }

    // ---- epilogue: out = round(round(acc) + bias), or acc -----------------
    const int ob = A.out_fmt == FMT_F32 ? 4 : 2;
    uint8_t* const og = A.out + bz * A.o_bs * ob;
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const int nblk = (wn >> 5) + b;  // row block of Bt in the tile
        const int n = n0 + 32 * nblk + ((lane & 31) ^ nblk);
        if (n >= A.N)
            continue;
        const bool has_bias = A.bias != nullptr;
        const float bv = has_bias ? A.bias[A.bias_len == 1 ? 0 : n] : 0.0f;
#pragma unroll
        for (int a = 0; a < 4; a++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int mblk = (wm >> 5) + a;
                const int m = m0 + 32 * mblk + ((8 * (i >> 2) + 4 * (lane >> 5) + (i & 3)) ^ mblk);
                if (m >= A.M)
                    continue;
                float r = acc[a][b][i];  // the file builds with -ffp-contract=off: no fused bias add
                if (has_bias)
                    r = round_fmt16(round_fmt16(r, A.out_fmt) + bv, A.out_fmt);
                const int64_t o = int64_t(m) * A.N + n;
                if (ob == 4)
                    reinterpret_cast<float*>(og)[o] = r;
                else
                    reinterpret_cast<uint16_t*>(og)[o] =
                        A.out_fmt == FMT_F16 ? f32_to_f16_bits(r) : f32_to_bf16_bits(r);
            }
        }
    }
}

constexpr int GLDS = 4 * GSTAGE;  // 128 KB

template <bool BF, bool KN>
void launch(const GemmF16Args& a, hipStream_t s)
{
    auto kfn = gemm_f16_kernel<BF, KN>;
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      GLDS),
                  "gemm_f16 LDS size");
        return true;
    }();
    (void)attr;
    const int tiles = a.batch * a.tiles_m * a.tiles_n;
    hipLaunchKernelGGL(kfn, dim3(unsigned(tiles)), dim3(GNT), GLDS, s, a);
}

}  // namespace

bool gemm_f16_supported(int64_t batch, int64_t m, int64_t n, int64_t k, bool b_kn, const void* a, const void* b)
{
    const bool aligned = (reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b)) % 16 == 0;
    const int64_t tiles = batch * ((m + GT - 1) / GT) * ((n + GT - 1) / GT);
    return aligned && k % GK == 0 && k > 0 && m > 0 && n > 0 && (!b_kn || n % 8 == 0) && tiles < (int64_t(1) << 31) &&
           m * k < (int64_t(1) << 31) && n * k < (int64_t(1) << 31) && m * n < (int64_t(1) << 31);
}

void gemm_f16(const GemmF16Desc& d, const void* a, const void* b, void* out, hipStream_t stream)
{
    GemmF16Args g{};
    g.a = static_cast<const uint16_t*>(a);
    g.b = static_cast<const uint16_t*>(b);
    g.out = static_cast<uint8_t*>(out);
    g.bias = static_cast<const float*>(d.bias);
    g.bias_len = d.bias_len;
    g.M = d.m;
    g.N = d.n;
    g.K = d.k;
    g.batch = d.batch;
    g.tiles_m = (d.m + GT - 1) / GT;
    g.tiles_n = (d.n + GT - 1) / GT;
    g.a_bs = int64_t(d.m) * d.k;
    g.b_bs = int64_t(d.n) * d.k;
    g.o_bs = int64_t(d.m) * d.n;
    g.out_fmt = d.out_fmt;
    const bool bf = d.elem == ELEM_BF16;
    if (bf) {
        if (d.b_kn)
            launch<true, true>(g, stream);
        else
            launch<true, false>(g, stream);
    } else {
        if (d.b_kn)
            launch<false, true>(g, stream);
        else
            launch<false, false>(g, stream);
    }
}

}  // namespace kern
}  // namespace tosa
