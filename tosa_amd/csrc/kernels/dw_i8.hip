// int8 DEPTHWISE_CONV2D (depth multiplier 1) on MFMA over an input tile
// staged in LDS, with the conv table's per-channel epilogue (bias,
// zero-point terms, RESCALE, CLAMP).
//
// Replaces Depthwise::accumulate::<AccI32> (src/ops/conv.rs:234-266), the
// bias add (src/ops/conv.rs:464) and, when fused, eval_rescale
// (src/ops/type_conv.rs:174-188) with apply_scale_32 (src/ops/quant.rs:17-32)
// and eval_clamp (src/ops/elementwise.rs:328-334).
//
// A workgroup owns R output rows (full width, every channel) of one image.
// It stages the input rows those outputs read -- (R - 1) sy + (KH - 1) dy + 1
// rows of (OW - 1) sx + (KW - 1) dx + 1 positions, positions outside the
// image holding the input zero point -- once, with coalesced 16-byte loads,
// and then every tap reads LDS. For 16 channels c0..c0+15 and 16 output pixels the depthwise sum
// out[c][p] = sum_t w[t][c] x~[p, t][c] is a 16 x 16 x 64 MFMA per four taps
// whose A operand is block-diagonal: lane (row c, k-chunk = tap t) holds
// w[t][c] in byte c of its 16 bytes and zero elsewhere; the B operand is the
// 16 channel bytes of (pixel, tap) read from LDS. The weight zero point's
// per-pixel term sum_t x~ comes from a second MFMA with ones on the diagonal.
// The (16-channel block, 16-pixel block) items of a tile are split into four
// contiguous runs, one per wave, channel-block major, so a wave rebuilds its
// weight fragments and table entries only when its run enters the next
// channel block.
#include <type_traits>

#include "kcommon.h"

namespace tosa {
namespace kern {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef unsigned v2u __attribute__((ext_vector_type(2)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lvoid;
typedef __attribute__((address_space(1))) void gvoid;

struct DwLdsArgs {
    const int8_t* x;
    const int8_t* w;
    const v4i* tab;     // conv table: 2 entries per channel
    uint8_t* out;
    uint32_t* err;
    int32_t C, IH, IW, OH, OW, KW, KH, T, sy, sx, dy, dx, pt, pl;
    // Tile rows, 16-byte channel chunks per position, LDS chunks per
    // position (nchk rounded up to odd: conflict-free fragment reads), halo
    // width, tiles per image.
    int32_t R, nchk, PS, HW, tiles_y;
    FastDiv div_ow, div_hw, div_nchk;
    int32_t zp_x, zp_w;
    int32_t clo, chi;  // output range narrowed to the CLAMP bounds
    int32_t range;     // some shift is below 32: check the value-range REQUIRE
};

template <int G, int OB, bool RS, bool ZW, bool RC>
__global__ void __launch_bounds__(256) dw_i8_lds_kernel(DwLdsArgs A)
{
    extern __shared__ v4u s_x[];  // [row][position][PS chunks], chunk q < nchk = channels 16q..16q+15
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j16 = lane & 15;
    const int grp = lane >> 4;

    const int ty = blockIdx.x % A.tiles_y;
    const int img = blockIdx.x / A.tiles_y;
    const int oy0 = ty * A.R;
    const int rows = A.OH - oy0 < A.R ? A.OH - oy0 : A.R;

    // ---- stage the input rows of the tile --------------------------------
    {
        const int iy0 = oy0 * A.sy - A.pt;
        const int hrows = (rows - 1) * A.sy + (A.KH - 1) * A.dy + 1;
        const int total = hrows * A.HW * A.nchk;
        const uint32_t zf = uint32_t(uint8_t(A.zp_x)) * 0x01010101u;
        const int8_t* xi = A.x + int64_t(img) * A.IH * A.IW * A.C;
        // U chunks per thread in flight at once: the loads are issued
        // together, then written to LDS. Consecutive threads read
        // consecutive 16-byte chunks of an input row.
        constexpr int U = 8;
        for (int i0 = tid; i0 < total; i0 += 256 * U) {
            v4u v[U];
            int dst[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int i = i0 + 256 * u;
                const int pos = fdiv(i, A.div_nchk);
                const int q = i - pos * A.nchk;
                const int hr = fdiv(pos, A.div_hw);
                const int hc = pos - hr * A.HW;
                const int iy = iy0 + hr, ix = hc - A.pl;
                const bool ok = i < total && unsigned(iy) < unsigned(A.IH) && unsigned(ix) < unsigned(A.IW);
                // Every lane loads (from the image origin when its position
                // is padding or past the tile) and then selects.
                const v4u ld = *reinterpret_cast<const v4u*>(
                    xi + (ok ? (int64_t(iy) * A.IW + ix) * A.C + 16 * q : int64_t(0)));
                v[u] = ok ? ld : v4u{zf, zf, zf, zf};
                dst[u] = pos * A.PS + q;
            }
#pragma unroll
            for (int u = 0; u < U; u++)
                if (i0 + 256 * u < total)
                    s_x[dst[u]] = v[u];
        }
    }
    __syncthreads();

    // ---- items (channel block, 16-pixel block), channel-block major; wave w
    // takes the w-th quarter, so its weights and table change at most a few
    // times.
    const int npx = rows * A.OW;
    const int nblk = (npx + 15) >> 4;
    const int items = A.nchk * nblk;
    const int lo = (items * wave) >> 2, hi_item = (items * (wave + 1)) >> 2;
    uint8_t* const out_img = A.out + (int64_t(img) * A.OH + oy0) * A.OW * int64_t(A.C) * OB;
    uint32_t bad_bits = 0;

    int cbk = -1, pb = 0;
    v4i wa[G], wo[G];
    int32_t toff[G];
    v4i t0[4], t1[4];
    int32_t hi[4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int t = 4 * g + grp;
        const bool tok = t < A.T;
        const int ky = t / A.KW, kx = t - (t / A.KW) * A.KW;
        toff[g] = tok ? ((ky * A.dy) * A.HW + kx * A.dx) * A.PS : 0;
        if constexpr (ZW) {
            // Ones on the block diagonal: sum_t x~ per pixel and channel.
            const int sh = 8 * (j16 & 3), wd = j16 >> 2;
            const uint32_t one = tok ? 1u : 0u;
            wo[g] = v4i{wd == 0 ? int(one << sh) : 0, wd == 1 ? int(one << sh) : 0, wd == 2 ? int(one << sh) : 0,
                        wd == 3 ? int(one << sh) : 0};
        }
    }
    for (int it = lo; it < hi_item; it++) {
        if (cbk < 0 || pb == nblk) {
            // First item, or the next channel block: its block-diagonal
            // weights (byte j16 of 16 is w[t][c0 + j16]) and table entries.
            cbk = cbk < 0 ? it / nblk : cbk + 1;
            pb = it - cbk * nblk;
            const int c0 = 16 * cbk;
#pragma unroll
            for (int g = 0; g < G; g++) {
                const int t = 4 * g + grp;
                const uint32_t wv = t < A.T ? uint32_t(uint8_t(A.w[t * A.C + c0 + j16])) : 0u;
                const int sh = 8 * (j16 & 3), wd = j16 >> 2;
                wa[g] = v4i{wd == 0 ? int(wv << sh) : 0, wd == 1 ? int(wv << sh) : 0,
                            wd == 2 ? int(wv << sh) : 0, wd == 3 ? int(wv << sh) : 0};
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                t0[i] = A.tab[2 * (c0 + 4 * grp + i)];
                if constexpr (RS)
                    t1[i] = A.tab[2 * (c0 + 4 * grp + i) + 1];
                hi[i] = ~t0[i].z;
            }
        }
        const int c0 = 16 * cbk;
        const int px = 16 * pb + j16;
        pb++;
        const bool valid = px < npx;
        const int pxc = valid ? px : 0;
        const int r = fdiv(pxc, A.div_ow);
        const int ox = pxc - r * A.OW;
        const int base = ((r * A.sy) * A.HW + ox * A.sx) * A.PS + cbk;
        v4i acc = v4i{0, 0, 0, 0}, acc1 = v4i{0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < G; g++) {
            const v4i bx = __builtin_bit_cast(v4i, s_x[base + toff[g]]);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[g], bx, acc, 0, 0, 0);
            if constexpr (ZW)
                acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(wo[g], bx, acc1, 0, 0, 0);
        }
        // Result element i of lane (grp, j16): channel c0 + 4 grp + i of
        // tile pixel j16.
        int32_t v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            uint32_t xu = uint32_t(acc[i]) + uint32_t(t0[i].x);
            if constexpr (ZW)
                xu += uint32_t(-A.zp_w) * uint32_t(acc1[i]);
            const int32_t xv = int32_t(xu);
            if constexpr (RS) {
                if constexpr (RC)
                    bad_bits = __builtin_amdgcn_bitop3_b32(bad_bits, uint32_t(med3_i32(xv, t0[i].z, hi[i])),
                                                           uint32_t(xv), 0xf6);  // bad | (med3 ^ x)
                const int64_t rp = __builtin_bit_cast(int64_t, v2i{t1[i].x, t1[i].y});
                const int64_t rn = __builtin_bit_cast(int64_t, v2i{t1[i].z, t1[i].w});
                const int32_t rr = int32_t((int64_t(xv) * int64_t(t0[i].y) + (xv >= 0 ? rp : rn)) >> t0[i].w);
                v[i] = med3_i32(rr, A.clo, A.chi);  // output zero point folded into rp, rn
            } else {
                v[i] = xv;
            }
        }
        if (valid) {
            uint8_t* dst = out_img + (int64_t(px) * A.C + c0 + 4 * grp) * OB;
            if constexpr (OB == 1)
                *reinterpret_cast<uint32_t*>(dst) = pack4_u8(v[0], v[1], v[2], v[3]);
            else if constexpr (OB == 2)
                *reinterpret_cast<v2u*>(dst) = v2u{__builtin_amdgcn_perm(uint32_t(v[1]), uint32_t(v[0]), 0x05040100u),
                                                   __builtin_amdgcn_perm(uint32_t(v[3]), uint32_t(v[2]), 0x05040100u)};
            else
                *reinterpret_cast<v4i*>(dst) = v4i{v[0], v[1], v[2], v[3]};
        }
        if constexpr (RS && RC)
            asm volatile("" : "+v"(bad_bits));
    }
    if (bad_bits)
        atomicOr(A.err, DERR_SCALE_RANGE);
}

constexpr int DW_LDS_MAX = 64 * 1024;
// Tile LDS aimed at: several workgroups per CU, so one stages while others
// compute.
constexpr int DW_LDS_TARGET = 24 * 1024;

template <int G, int OB, bool RS, bool ZW, bool RC>
void launch(const DwLdsArgs& a, unsigned blocks, size_t lds, hipStream_t s)
{
    auto kfn = dw_i8_lds_kernel<G, OB, RS, ZW, RC>;
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      DW_LDS_MAX),
                  "depthwise LDS size");
        return true;
    }();
    (void)attr;
    hipLaunchKernelGGL(kfn, dim3(blocks), dim3(256), lds, s, a);
}

template <int G>
void launch_epi(const DwLdsArgs& a, unsigned blocks, size_t lds, int ob, bool rs, bool zw, hipStream_t s)
{
    if (!rs) {
        if (zw)
            launch<G, 4, false, true, false>(a, blocks, lds, s);
        else
            launch<G, 4, false, false, false>(a, blocks, lds, s);
        return;
    }
#define TOSA_DW_RC(OBV, ZWV)                                  \
    if (a.range)                                              \
        launch<G, OBV, true, ZWV, true>(a, blocks, lds, s);   \
    else                                                      \
        launch<G, OBV, true, ZWV, false>(a, blocks, lds, s);
#define TOSA_DW_OB(OBV)      \
    if (zw) {                \
        TOSA_DW_RC(OBV, true) \
    } else {                 \
        TOSA_DW_RC(OBV, false) \
    }
    if (ob == 1) {
        TOSA_DW_OB(1)
    } else if (ob == 2) {
        TOSA_DW_OB(2)
    } else {
        TOSA_DW_OB(4)
    }
#undef TOSA_DW_OB
#undef TOSA_DW_RC
}


// ---------------------------------------------------------------------------
// Pipelined variant: persistent workgroups over (image, R output rows, CB
// channels) tiles. A tile's input rows, its channels' weights and table
// entries are fetched by direct global -> LDS loads (each load instruction
// fills 1 KB of LDS from 16-byte pieces: no per-tap scattered reads through
// the L1) into one of two buffers while the workgroup computes the previous
// tile from the other. Tiles are numbered channel chunk fastest, then rows,
// then image; each round of gridDim.x tiles gives every XCD a contiguous run
// of them, so tiles that share input halo rows or output cache lines meet in
// one L2.
struct DwPipeArgs {
    const int8_t* x;
    const int8_t* w;
    const v4i* tab;
    const int8_t* zfill;  // 16 bytes of the input zero point
    uint8_t* out;
    uint32_t* err;
    int32_t C, IH, IW, OH, OW, KW, KH, T, sy, sx, dy, dx, pt, pl;
    // Channels per tile and their 16-byte chunks, LDS chunks per position
    // (nq rounded up to odd: conflict-free fragment reads), tile rows, input
    // rows and positions per tile, tiles along the height, channel chunks,
    // tiles in all.
    int32_t CB, nq, PS, R, HR, HW, tiles_y, nchunks, units;
    int32_t tslots;  // 16-byte slots of the input rows (HR x HW x PS)
    int32_t slots;   // slots of a buffer: input, weights [T][CB], table [CB][2]; a multiple of 64
    FastDiv div_ow, div_hw, div_ps, div_nq, div_nch, div_ty;
    float inv_ow, hinv_ow;  // 1 / OW and 0.5 / OW (the tile's row of a pixel)
    int32_t negow;          // -OW
    int32_t rstep, xstep;   // LDS bytes per output row (16 sy HW PS) and per output column (16 sx PS)
    int32_t zp_w;
    int32_t clo, chi;
    int32_t range;
};

template <int G, int OB, bool RS, bool ZW, bool RC>
__global__ void __launch_bounds__(512) dw_i8_pipe_kernel(DwPipeArgs A)
{
    extern __shared__ v4u s_buf[];  // two buffers of A.slots 16-byte slots
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int j16 = lane & 15;
    const int grp = lane >> 4;
    // Tile of round k: workgroup b runs on XCD b % 8 and takes place b / 8
    // of that XCD's run (gridDim.x is a multiple of 8).
    const int per_xcd = gridDim.x >> 3;
    const int first = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    auto unit_of = [&](int k) { return k * int(gridDim.x) + first; };
    auto decode = [&](int u, int& img, int& oy0, int& c0) {
        const int rest = fdiv(u, A.div_nch);
        c0 = (u - rest * A.nchunks) * A.CB;
        img = fdiv(rest, A.div_ty);
        oy0 = (rest - img * A.tiles_y) * A.R;
    };
    // Slot s of a buffer: input chunk (position s / PS, chunk s % PS; chunks
    // past nq and positions outside the image load the zero-point fill),
    // then the weights w[t][c0 + 16 q ..], then the table entries of the
    // tile's channels; slots past those load the fill into padding.
    auto dma = [&](int u, int buf) {
        int img, oy0, c0;
        decode(u, img, oy0, c0);
        const int iy0 = oy0 * A.sy - A.pt;
        const int8_t* const xi = A.x + int64_t(img) * A.IH * A.IW * A.C + c0;
        const int wslots = A.T * A.nq;
        v4u* const dst = s_buf + buf * A.slots;
        for (int s0 = wave * 64; s0 < A.slots; s0 += 512) {
            const int s = s0 + lane;
            const int8_t* src = A.zfill;
            if (s < A.tslots) {
                const int hp = fdiv(s, A.div_ps);
                const int q = s - hp * A.PS;
                const int hr = fdiv(hp, A.div_hw);
                const int iy = iy0 + hr, ix = hp - hr * A.HW - A.pl;
                if (q < A.nq && unsigned(iy) < unsigned(A.IH) && unsigned(ix) < unsigned(A.IW))
                    src = xi + (int64_t(iy) * A.IW + ix) * A.C + 16 * q;
            } else if (s < A.tslots + wslots) {
                const int s2 = s - A.tslots;
                const int t = fdiv(s2, A.div_nq);
                src = A.w + t * A.C + c0 + 16 * (s2 - t * A.nq);
            } else if (s < A.tslots + wslots + 2 * A.CB) {
                src = reinterpret_cast<const int8_t*>(A.tab + 2 * c0 + (s - A.tslots - wslots));
            }
            __builtin_amdgcn_global_load_lds((gvoid*)src, (lvoid*)(dst + s0), 16, 0, 0);
        }
    };

    // Tap offsets inside a tile (LDS bytes) of this lane's k-chunk in each
    // group, and the block-diagonal -zw of the weight zero point's term,
    // which accumulates into the same chain: sum_t (w - zw) x~.
    int32_t toff[G];  // bytes
    v4i wo[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int t = 4 * g + grp;
        const bool tok = t < A.T;
        const int ky = t / A.KW, kx = t - (t / A.KW) * A.KW;
        toff[g] = tok ? ((ky * A.dy) * A.HW + kx * A.dx) * A.PS * 16 : 0;
        if constexpr (ZW) {
            const int sh = 8 * (j16 & 3), wd = j16 >> 2;
            const uint32_t nz = tok ? uint32_t(uint8_t(-A.zp_w)) : 0u;  // zw != -128
            wo[g] = v4i{wd == 0 ? int(nz << sh) : 0, wd == 1 ? int(nz << sh) : 0, wd == 2 ? int(nz << sh) : 0,
                        wd == 3 ? int(nz << sh) : 0};
        }
    }
    uint32_t bad_bits = 0;
    // Clamp bounds held in VGPRs for the whole kernel (v_med3 takes one
    // scalar operand at most).
    int32_t vclo, vchi;
    asm volatile("v_mov_b32 %0, %1" : "=v"(vclo) : "s"(A.clo));
    asm volatile("v_mov_b32 %0, %1" : "=v"(vchi) : "s"(A.chi));

    if (first < A.units)
        dma(first, 0);
    for (int k = 0;; k++) {
        const int u = unit_of(k);
        if (u >= A.units)
            break;
        // This tile's loads have landed, and every wave is done with the
        // buffer that the next tile's loads overwrite.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (unit_of(k + 1) < A.units)
            dma(unit_of(k + 1), (k + 1) & 1);

        int img, oy0, c0;
        decode(u, img, oy0, c0);
        const int rows = A.OH - oy0 < A.R ? A.OH - oy0 : A.R;
        const int npx = rows * A.OW;
        const int nblk = (npx + 31) >> 5;
        const int items = A.nq * nblk;
        // Items (16-channel block q, 32-pixel block: two independent 16-pixel
        // MFMA chains), block major; wave w takes the w-th eighth, so its
        // fragments change a few times.
        const int lo = (items * wave) >> 3, hi_item = (items * (wave + 1)) >> 3;
        const v4u* const sx = s_buf + (k & 1) * A.slots;
        const uint8_t* const sw = reinterpret_cast<const uint8_t*>(sx + A.tslots);
        const v4i* const st = reinterpret_cast<const v4i*>(sx + A.tslots + A.T * A.nq);
        uint8_t* const out0 = A.out + ((int64_t(img) * A.OH + oy0) * A.OW * A.C + c0) * OB;
        int q = -1, pb = 0;
        v4i wa[G], t0[4], add;
        int64_t rp[4], rn[4];
        int32_t hi[4];
        for (int it = lo; it < hi_item; it++) {
            if (q < 0 || pb == nblk) {
                q = q < 0 ? it / nblk : q + 1;
                pb = it - q * nblk;
                // Block-diagonal weights (byte j16 of 16 is w[t][16 q + j16])
                // and the table entries of the lane's channels 16 q + 4 grp + i.
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const int t = 4 * g + grp;
                    const uint32_t wv = t < A.T ? uint32_t(sw[t * A.CB + 16 * q + j16]) : 0u;
                    const int sh = 8 * (j16 & 3), wd = j16 >> 2;
                    wa[g] = v4i{wd == 0 ? int(wv << sh) : 0, wd == 1 ? int(wv << sh) : 0,
                                wd == 2 ? int(wv << sh) : 0, wd == 3 ? int(wv << sh) : 0};
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    t0[i] = st[2 * (16 * q + 4 * grp + i)];
                    if constexpr (RS) {
                        const v4i t1 = st[2 * (16 * q + 4 * grp + i) + 1];
                        rp[i] = __builtin_bit_cast(int64_t, v2i{t1.x, t1.y});
                        rn[i] = __builtin_bit_cast(int64_t, v2i{t1.z, t1.w});
                    }
                    hi[i] = ~t0[i].z;
                }
                // The chains start at the channels' additive constants.
                add = v4i{t0[0].x, t0[1].x, t0[2].x, t0[3].x};
            }
            const char* const sxq = reinterpret_cast<const char*>(sx + q);
            int px[2];
            v4i acc[2];
#pragma unroll
            for (int b = 0; b < 2; b++) {
                px[b] = 32 * pb + 16 * b + j16;
                const int pxc = px[b] < npx ? px[b] : 0;
                // Row of the tile pixel: pxc / OW rounded down, exact for
                // pixels below 2^15 and widths up to 4096 (tiles hold fewer
                // than 2600 pixels).
                const int r = int(__builtin_fmaf(float(pxc), A.inv_ow, A.hinv_ow));
                const int ox = __mul24(r, A.negow) + pxc;
                const int base = __mul24(r, A.rstep) + __mul24(ox, A.xstep);  // bytes
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const v4i bx = *reinterpret_cast<const v4i*>(sxq + base + toff[g]);
                    acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[g], bx, g == 0 ? add : acc[b], 0, 0, 0);
                    if constexpr (ZW)
                        acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wo[g], bx, acc[b], 0, 0, 0);
                }
            }
            pb++;
            // Result element i of lane (grp, j16) in chain b: channel
            // 16 q + 4 grp + i of tile pixel 32 pb + 16 b + j16.
#pragma unroll
            for (int b = 0; b < 2; b++) {
                int32_t v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int32_t xv = acc[b][i];
                    if constexpr (RS) {
                        // (Plain min/max here: the value comes straight from
                        // the MFMA, whose result hazards the compiler tracks
                        // only for instructions it emits itself.)
                        if constexpr (RC)
                            bad_bits |= uint32_t(std::min(std::max(xv, t0[i].z), hi[i]) ^ xv);
                        const int32_t rr = int32_t((int64_t(xv) * int64_t(t0[i].y) + (xv >= 0 ? rp[i] : rn[i])) >> t0[i].w);
                        v[i] = med3_i32(rr, vclo, vchi);  // output zero point folded into rp, rn
                    } else {
                        v[i] = xv;
                    }
                }
                if (px[b] < npx) {
                    uint8_t* dst = out0 + uint32_t(__mul24(px[b], A.C * OB) + (16 * q + 4 * grp) * OB);
                    if constexpr (OB == 1)
                        *reinterpret_cast<uint32_t*>(dst) = pack4_u8(v[0], v[1], v[2], v[3]);
                    else if constexpr (OB == 2)
                        *reinterpret_cast<v2u*>(dst) =
                            v2u{__builtin_amdgcn_perm(uint32_t(v[1]), uint32_t(v[0]), 0x05040100u),
                                __builtin_amdgcn_perm(uint32_t(v[3]), uint32_t(v[2]), 0x05040100u)};
                    else
                        *reinterpret_cast<v4i*>(dst) = v4i{v[0], v[1], v[2], v[3]};
                }
                if constexpr (RS && RC)
                    asm volatile("" : "+v"(bad_bits));
            }
        }
    }
    if (bad_bits)
        atomicOr(A.err, DERR_SCALE_RANGE);
}

constexpr int DW_PIPE_BUF_MAX = 40 * 1024;

template <int G, int OB, bool RS, bool ZW, bool RC>
void launch_pipe(const DwPipeArgs& a, unsigned blocks, size_t lds, hipStream_t s)
{
    auto kfn = dw_i8_pipe_kernel<G, OB, RS, ZW, RC>;
    static bool attr = [&]() {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kfn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      2 * DW_PIPE_BUF_MAX),
                  "depthwise pipeline LDS size");
        return true;
    }();
    (void)attr;
    hipLaunchKernelGGL(kfn, dim3(blocks), dim3(512), lds, s, a);
}

template <int G>
void launch_pipe_epi(const DwPipeArgs& a, unsigned blocks, size_t lds, int ob, bool rs, bool zw, hipStream_t s)
{
    if (!rs) {
        if (zw)
            launch_pipe<G, 4, false, true, false>(a, blocks, lds, s);
        else
            launch_pipe<G, 4, false, false, false>(a, blocks, lds, s);
        return;
    }
#define TOSA_DWP_RC(OBV, ZWV)                                      \
    if (a.range)                                                   \
        launch_pipe<G, OBV, true, ZWV, true>(a, blocks, lds, s);   \
    else                                                           \
        launch_pipe<G, OBV, true, ZWV, false>(a, blocks, lds, s);
#define TOSA_DWP_OB(OBV)        \
    if (zw) {                   \
        TOSA_DWP_RC(OBV, true)  \
    } else {                    \
        TOSA_DWP_RC(OBV, false) \
    }
    if (ob == 1) {
        TOSA_DWP_OB(1)
    } else if (ob == 2) {
        TOSA_DWP_OB(2)
    } else {
        TOSA_DWP_OB(4)
    }
#undef TOSA_DWP_OB
#undef TOSA_DWP_RC
}

}  // namespace

bool depthwise_i8_lds(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                      hipStream_t stream)
{
    const int T = d.kh * d.kw;
    if (!d.depthwise || d.ic % 16 != 0 || T > 12 || d.oc != d.ic || reinterpret_cast<uintptr_t>(d.x) % 16 != 0)
        return false;
    // Images below 28 x 28 leave too few tiles with every channel in one
    // workgroup; the direct-load kernel does better there.
    if (int64_t(d.ih) * d.iw < 28 * 28)
        return false;
    DwLdsArgs a{};
    a.x = d.x;
    a.w = d.w;
    a.tab = static_cast<const v4i*>(tab);
    a.out = static_cast<uint8_t*>(out);
    a.err = err;
    a.C = d.ic;
    a.IH = d.ih;
    a.IW = d.iw;
    a.OH = d.oh;
    a.OW = d.ow;
    a.KW = d.kw;
    a.KH = d.kh;
    a.T = T;
    a.sy = d.sy;
    a.sx = d.sx;
    a.dy = d.dy;
    a.dx = d.dx;
    a.pt = d.pt;
    a.pl = d.pl;
    a.zp_x = d.zp_x;
    a.zp_w = d.zp_w;
    int ob = 4;
    if (rs) {
        a.clo = int32_t(rs->has_clamp ? std::max<int64_t>(rs->clamp_lo, rs->lo) : rs->lo);
        a.chi = int32_t(rs->has_clamp ? std::min<int64_t>(rs->clamp_hi, rs->hi) : rs->hi);
        a.range = rs->min_shift <= 31 && !d.range_safe;
        ob = rs->out_bytes;
    }
    // The workgroup owns every channel of its pixels: coalesced staging,
    // and each output line is written by one workgroup.
    a.nchk = d.ic / 16;
    a.PS = a.nchk | 1;
    a.HW = (d.ow - 1) * d.sx + (d.kw - 1) * d.dx + 1;
    // Rows per tile: about 512 output pixels, within the LDS target, and
    // fewer when the grid would not cover the chip a few times over.
    auto lds_for = [&](int r) { return size_t((r - 1) * d.sy + (d.kh - 1) * d.dy + 1) * a.HW * a.PS * 16; };
    int R = std::max(1, std::min(d.oh, 512 / std::max(1, d.ow)));
    while (R > 1 && lds_for(R) > size_t(DW_LDS_TARGET))
        R--;
    if (lds_for(R) > size_t(DW_LDS_MAX))
        return false;
    auto blocks_for = [&](int r) { return int64_t(d.n) * ((d.oh + r - 1) / r); };
    while (R > 1 && blocks_for(R) < 1024)
        R = (R + 1) / 2;
    a.R = R;
    a.tiles_y = (d.oh + R - 1) / R;
    a.div_ow = FastDiv(uint32_t(d.ow));
    a.div_hw = FastDiv(uint32_t(a.HW));
    a.div_nchk = FastDiv(uint32_t(a.nchk));
    const int64_t blocks = blocks_for(R);
    if (blocks <= 0 || blocks >= (int64_t(1) << 31))
        return false;
    const size_t lds = lds_for(R);
    const int groups = (T + 3) / 4;
    const bool zw = d.zp_w != 0;
    if (groups == 1)
        launch_epi<1>(a, unsigned(blocks), lds, ob, rs != nullptr, zw, stream);
    else if (groups == 2)
        launch_epi<2>(a, unsigned(blocks), lds, ob, rs != nullptr, zw, stream);
    else
        launch_epi<3>(a, unsigned(blocks), lds, ob, rs != nullptr, zw, stream);
    return true;
}

namespace {

// Launches the pipelined kernel with tiles of 16 nq channels x R output
// rows; false when the tile's buffer exceeds the LDS budget.
bool dw_pipe_launch(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err, int nq,
                    int R, hipStream_t stream)
{
    const int T = d.kh * d.kw;
    // The weight zero point rides in the MFMA as the int8 -zw.
    if (nq <= 0 || (d.ic / 16) % nq != 0 || R <= 0 || d.ow > 4096 || d.zp_w == -128)
        return false;
    DwPipeArgs a{};
    const int HW = (d.ow - 1) * d.sx + (d.kw - 1) * d.dx + 1;
    a.x = d.x;
    a.w = d.w;
    a.tab = static_cast<const v4i*>(tab);
    a.zfill = reinterpret_cast<const int8_t*>(a.tab + 2 * d.oc);
    a.out = static_cast<uint8_t*>(out);
    a.err = err;
    a.C = d.ic;
    a.IH = d.ih;
    a.IW = d.iw;
    a.OH = d.oh;
    a.OW = d.ow;
    a.KW = d.kw;
    a.KH = d.kh;
    a.T = T;
    a.sy = d.sy;
    a.sx = d.sx;
    a.dy = d.dy;
    a.dx = d.dx;
    a.pt = d.pt;
    a.pl = d.pl;
    a.zp_w = d.zp_w;
    int ob = 4;
    if (rs) {
        a.clo = int32_t(rs->has_clamp ? std::max<int64_t>(rs->clamp_lo, rs->lo) : rs->lo);
        a.chi = int32_t(rs->has_clamp ? std::min<int64_t>(rs->clamp_hi, rs->hi) : rs->hi);
        a.range = rs->min_shift <= 31 && !d.range_safe;
        ob = rs->out_bytes;
    }
    a.nq = nq;
    a.R = R;
    a.CB = 16 * a.nq;
    a.PS = a.nq | 1;
    a.HR = (a.R - 1) * d.sy + (d.kh - 1) * d.dy + 1;
    a.HW = HW;
    a.tiles_y = (d.oh + a.R - 1) / a.R;
    a.nchunks = d.ic / a.CB;
    const int64_t units = int64_t(d.n) * a.tiles_y * a.nchunks;
    if (units >= (int64_t(1) << 30) || int64_t(d.n) * d.ih * d.iw * d.ic >= (int64_t(1) << 40))
        return false;
    a.units = int32_t(units);
    a.tslots = a.HR * a.HW * a.PS;
    a.slots = (a.tslots + T * a.nq + 2 * a.CB + 63) / 64 * 64;
    if (size_t(a.slots) * 16 > size_t(DW_PIPE_BUF_MAX))
        return false;
    a.div_ow = FastDiv(uint32_t(d.ow));
    a.div_hw = FastDiv(uint32_t(a.HW));
    a.div_ps = FastDiv(uint32_t(a.PS));
    a.div_nq = FastDiv(uint32_t(a.nq));
    a.div_nch = FastDiv(uint32_t(a.nchunks));
    a.div_ty = FastDiv(uint32_t(a.tiles_y));
    a.inv_ow = 1.0f / float(d.ow);
    a.hinv_ow = 0.5f / float(d.ow);
    a.negow = -d.ow;
    a.rstep = 16 * d.sy * a.HW * a.PS;
    a.xstep = 16 * d.sx * a.PS;
    const size_t lds = size_t(2) * a.slots * 16;
    const long wpc = std::min<long>(2, (160L * 1024) / long(lds));
    // A multiple of 8 workgroups (the tile order deals runs to the 8 XCDs).
    const int64_t grid = std::min<int64_t>(int64_t(cu_count()) * wpc, (units + 7) / 8 * 8);
    const unsigned blocks = unsigned((grid + 7) / 8 * 8);
    const int groups = (T + 3) / 4;
    const bool zw = d.zp_w != 0;
    if (groups == 1)
        launch_pipe_epi<1>(a, blocks, lds, ob, rs != nullptr, zw, stream);
    else if (groups == 2)
        launch_pipe_epi<2>(a, blocks, lds, ob, rs != nullptr, zw, stream);
    else
        launch_pipe_epi<3>(a, blocks, lds, ob, rs != nullptr, zw, stream);
    return true;
}


}  // namespace

bool depthwise_i8_pipe(const ConvI8Desc& d, const void* tab, const RescaleDev* rs, void* out, uint32_t* err,
                       hipStream_t stream)
{
    const int T = d.kh * d.kw;
    const bool aligned = (reinterpret_cast<uintptr_t>(d.x) | reinterpret_cast<uintptr_t>(d.w)) % 16 == 0;
    if (!d.depthwise || d.ic % 16 != 0 || T > 12 || d.oc != d.ic || !aligned || d.n <= 0 || d.oh <= 0 ||
        d.ow <= 0)
        return false;
    const int HW = (d.ow - 1) * d.sx + (d.kw - 1) * d.dx + 1;
    const int obytes = rs ? rs->out_bytes : 4;
    // Tile shape: channel chunks CB (a divisor of C in 16-channel steps) and
    // rows R whose two buffers fit, picked by the bytes the busiest CU
    // moves: tiles per CU (whole rounds of the persistent grid) x (loaded
    // input rows + weights + table + written outputs + a fixed cost per
    // tile). Halo rows count as loaded even where L2 serves them. A sweep of
    // every shape on MobileNetV2's ten depthwise layers put this pick within
    // 10 % of the fastest shape on each.
    const long cus = cu_count();
    const int nch16 = d.ic / 16;
    long best = -1;
    int bnq = 0, bR = 0;
    for (int nq = 1; nq <= nch16; nq++) {
        if (nch16 % nq != 0)
            continue;
        const int PS = nq | 1;
        for (int R = 1; R <= d.oh; R++) {
            const long HR = long(R - 1) * d.sy + long(d.kh - 1) * d.dy + 1;
            const long tsl = HR * HW * PS;
            const long slots = (tsl + long(T) * nq + 32L * nq + 63) / 64 * 64;
            if (slots * 16 > DW_PIPE_BUF_MAX)
                break;
            const long wpc = std::min<long>(2, (160L * 1024) / (2 * slots * 16));
            const long tiles_y = (d.oh + R - 1) / R;
            const long units = long(d.n) * tiles_y * (nch16 / nq);
            const long grid = cus * wpc;
            const long per_cu = (units + grid - 1) / grid * wpc;
            // Narrow chunks cost more than their bytes: with one 16-byte chunk
            // per position every load lane reads a different pixel (measured
            // on a 112 x 112 x 96 stride-2 layer: 48-channel tiles 28 us,
            // 16-channel tiles 33 us), charged here as half a chunk's bytes
            // again over nq.
            const long tile_bytes = tsl * 16 + tsl * 8 / nq + long(R) * d.ow * 16 * nq * obytes + 4096;
            const long cost = per_cu * tile_bytes;
            if (best < 0 || cost < best) {
                best = cost;
                bnq = nq;
                bR = R;
            }
        }
    }
    if (best < 0)
        return false;
    return dw_pipe_launch(d, tab, rs, out, err, bnq, bR, stream);
}

}  // namespace kern
}  // namespace tosa
