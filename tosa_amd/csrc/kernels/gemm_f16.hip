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
// 6 fragment reads per 8 MFMAs), K staged 32 elements at a time through a
// ring of four LDS buffers with the direct global->LDS loads of three stages
// in flight. LDS image of an A (or [N][K] B) stage: the 16-byte chunk holding
// elements 16 j + 8 c .. + 7 of row r (block b = r / 32 of the tile) sits at
// slot ((8 j + b) 2 + c) 32 + ((r % 32) ^ b), so the fragment read of a row
// block (lane l: k-half l / 32) is one contiguous 1 KB, and lane l holds row
// 32 b + ((l % 32) ^ b); the epilogue undoes that permutation.
// A [K][N] B stage is copied as it lies: row k of the stage (256 columns, 32
// 16-byte pieces) with piece p stored at p ^ (4 k % 32), and its fragments
// are read with the LDS transpose read ds_read_b64_tr_b16: in each group of
// 16 lanes, lane i receives element i % 4 of the 8-byte pieces addressed by
// lanes i / 4 + 4 j (j = 0..3); lane s addresses row k0 + s / 4, columns
// nb + 4 (s % 4), so lane i gets column nb + i of rows k0 .. k0 + 3 (the XOR
// places the four rows and two column halves a 16-lane group reads in
// distinct bank groups).
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
constexpr int GK = 32;         // K elements per stage
constexpr int GNT = 512;       // threads
constexpr int GSTAGE = GT * GK * 2;  // bytes of one operand stage (16 KB)
constexpr int GNS = 4;         // stages in the LDS ring
static_assert(GNS - 2 <= 6, "vmcnt cases");

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
// assembly so that the compiler's wait counting, which would drain every
// such load before any LDS read, leaves the fragment reads alone; the kernel
// counts these loads itself (s_waitcnt vmcnt) before the barrier that
// precedes a stage's reads.
__device__ __forceinline__ void dma16(const void* g, const void* l)
{
    const uint32_t la = __builtin_amdgcn_readfirstlane(uint32_t(reinterpret_cast<uintptr_t>((const lvoid*)l)));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(la) : "memory", "m0");
}

typedef short v4s __attribute__((ext_vector_type(4)));
// Transposing 8-byte LDS read (see the layout note above).
__device__ __forceinline__ v2u ldtr16(const uint8_t* p)
{
    const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)((const lvoid*)p));
    return __builtin_bit_cast(v2u, r);
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
    uint8_t* const sA = smem;                  // [GNS][GSTAGE]
    uint8_t* const sB = smem + GNS * GSTAGE;   // [GNS][GSTAGE]

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

    // ---- staging: GSTAGE / 1024 = 16 loads of 1 KB per operand, two per wave
    // DMA q fills slots 64 q .. + 63: k16 step j = q / 8, row block b = q % 8,
    // rows 32 b + ((l % 32) ^ b), k-half l / 32. Rows past the matrix re-read
    // its last row (their results are not stored).
    auto dma_rows = [&](const uint16_t* g, int rows, int r0, int k0, uint8_t* dst) {
#pragma unroll
        for (int i = 0; i < GSTAGE / 1024 / (GNT / 64); i++) {
            const int q = wave + (GNT / 64) * i;
            const int j = q >> 3, row = 32 * (q & 7) + ((lane & 31) ^ (q & 7)), c = lane >> 5;
            const int r = r0 + row < rows ? r0 + row : rows - 1;
            dma16(g + int64_t(r) * A.K + k0 + 16 * j + 8 * c, dst + q * 1024);
        }
    };
    // [K][N] B: DMA q fills rows 2 q, 2 q + 1 of the stage; lane l writes
    // piece l % 32 of row 2 q + l / 32, which holds the row's piece
    // (l % 32) ^ (4 row % 32). Pieces past N re-read column 0 (those
    // columns are not stored).
    auto dma_kn = [&](int k0, uint8_t* dst) {
#pragma unroll
        for (int i = 0; i < GSTAGE / 1024 / (GNT / 64); i++) {
            const int q = wave + (GNT / 64) * i;
            const int row = 2 * q + (lane >> 5);
            const int piece = (lane & 31) ^ ((4 * row) & 31);
            const int n = n0 + 8 * piece;
            dma16(bg + int64_t(k0 + row) * A.N + (n < A.N ? n : 0), dst + q * 1024);
        }
    };
    auto issue = [&](int st) {
        const int slot = st % GNS;
        dma_rows(ag, A.M, m0, st * GK, sA + slot * GSTAGE);
        if constexpr (KN)
            dma_kn(st * GK, sB + slot * GSTAGE);
        else
            dma_rows(bg, A.N, n0, st * GK, sB + slot * GSTAGE);
    };

    // ---- waves: 2 (M) x 4 (N), each 128 x 64 ------------------------------
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
    v16f acc[4][2];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
            acc[a][b] = v16f{};

    // Fragment of rows r0 .. r0 + 31 (r0 % 32 == 0) for k16 step j: one
    // contiguous 1 KB.
    auto frag = [&](const uint8_t* base, int j, int r0) {
        return *reinterpret_cast<const v4u*>(base + (8 * j + (r0 >> 5)) * 1024 + lane * 16);
    };
    // [K][N] B fragment of columns c0 .. c0 + 31 for k16 step j: lane l gets
    // column c0 + l % 32, elements 16 j + 8 (l / 32) .. + 7 (two transposing
    // reads of four rows each).
    const int trs = lane & 15, trg = lane >> 4;
    auto frag_kn = [&](const uint8_t* base, int j, int c0) {
        v2u h[2];
#pragma unroll
        for (int sub = 0; sub < 2; sub++) {
            const int row = 16 * j + 8 * (trg >> 1) + 4 * sub + (trs >> 2);
            const int col = c0 + 16 * (trg & 1) + 4 * (trs & 3);  // element column in the tile
            const int piece = (col >> 3) ^ ((4 * row) & 31);
            h[sub] = ldtr16(base + row * (GT * 2) + piece * 16 + (col & 7) * 2);
        }
        return v4u{h[0].x, h[0].y, h[1].x, h[1].y};
    };

    const int nst = A.K / GK;
    // GNS - 1 stages in flight; stage st's loads are the oldest outstanding
    // ones when the wave waits for them.
    constexpr int LPS = 2 * GSTAGE / 1024 / (GNT / 64);  // loads per stage and wave
#pragma unroll
    for (int st = 0; st < GNS - 1; st++)
        if (st < nst)
            issue(st);
    for (int st = 0; st < nst; st++) {
        // vmcnt(N): at most N of this wave's loads outstanding, those of the
        // later stages already issued (gfx9 s_waitcnt: vmcnt in bits 3-0 and
        // 15-14, expcnt 6-4 and lgkmcnt 11-8 left at their maxima).
        const int later = nst - 1 - st < GNS - 2 ? nst - 1 - st : GNS - 2;
        switch (later) {
#define TOSA_WAIT_VM(L)                                                                   \
    case L:                                                                               \
        __builtin_amdgcn_s_waitcnt(0x0F70 | ((L * LPS) & 15) | (((L * LPS) >> 4) << 14)); \
        break;
            TOSA_WAIT_VM(0)
            TOSA_WAIT_VM(1)
            TOSA_WAIT_VM(2)
            TOSA_WAIT_VM(3)
            TOSA_WAIT_VM(4)
            TOSA_WAIT_VM(5)
            TOSA_WAIT_VM(6)
#undef TOSA_WAIT_VM
        default:
            __builtin_amdgcn_s_waitcnt(0x0F70);
        }
        // Every wave's loads of stage st have landed, and every wave is done
        // with the buffer that stage st + GNS - 1 overwrites (stage st - 1's).
        __syncthreads();
        if (st + GNS - 1 < nst)
            issue(st + GNS - 1);
        const uint8_t* const a_s = sA + (st % GNS) * GSTAGE;
        const uint8_t* const b_s = sB + (st % GNS) * GSTAGE;
#pragma unroll
        for (int j = 0; j < GK / 16; j++) {
            v4u fa[4], fb[2];
#pragma unroll
            for (int a = 0; a < 4; a++)
                fa[a] = frag(a_s, j, wm + 32 * a);
#pragma unroll
            for (int b = 0; b < 2; b++) {
                if constexpr (KN)
                    fb[b] = frag_kn(b_s, j, wn + 32 * b);
                else
                    fb[b] = frag(b_s, j, wn + 32 * b);
            }
#pragma unroll
            for (int b = 0; b < 2; b++)
#pragma unroll
                for (int a = 0; a < 4; a++)
                    acc[a][b] = mfma32<BF>(fa[a], fb[b], acc[a][b]);
        }
    }

    // ---- epilogue: out = round(round(acc) + bias), or acc -----------------
    const int ob = A.out_fmt == FMT_F32 ? 4 : 2;
    uint8_t* const og = A.out + bz * A.o_bs * ob;
#pragma unroll
    for (int b = 0; b < 2; b++) {
        const int nblk = (wn >> 5) + b;  // row block of Bt in the tile
        const int n = n0 + 32 * nblk + (KN ? (lane & 31) : ((lane & 31) ^ nblk));
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

constexpr int GLDS = 2 * GNS * GSTAGE;  // 128 KB

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
