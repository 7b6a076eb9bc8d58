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

}  // namespace kern
}  // namespace tosa
