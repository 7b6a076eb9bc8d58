// Bandwidth-bound kernels: int8 DEPTHWISE_CONV2D, AVG_POOL2D, MAX_POOL2D,
// RESCALE, CAST, CLAMP, ADD, the fused quantised residual add, TRANSPOSE,
// and the int16 split / INT48 assembly around the int8 MFMA kernels.
#include "kcommon.h"

#pragma clang fp contract(off)

namespace tosa {
namespace kern {
namespace {

// Bytes j of four words gathered into one word: [x0.bj, x1.bj, x2.bj, x3.bj].
__device__ __forceinline__ uint32_t gather_byte(uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3, int j)
{
    const int s = 8 * j;
    return ((x0 >> s) & 0xFFu) | (((x1 >> s) & 0xFFu) << 8) | (((x2 >> s) & 0xFFu) << 16) | (((x3 >> s) & 0xFFu) << 24);
}

// ---------------------------------------------------------------------------
// int8 DEPTHWISE_CONV2D, depth multiplier 1, KH*KW <= 12 taps.
//
// Replaces Depthwise::accumulate (src/ops/conv.rs:234-266) for int8. A thread
// owns 4 consecutive channels of PX consecutive output pixels in a row. Taps
// are grouped four at a time and transposed so that one v_dot4_i32_i8 sums
// four taps of one channel; zero points are folded exactly as in the
// implicit GEMM: sum (x~ - zx)(w - zw) = sum x~ w - zw sum x~ - zx sum w +
// T zx zw, with padding taps loaded as zx.
// ---------------------------------------------------------------------------
template <int KH, int KW, int PX>
__global__ void __launch_bounds__(256) dw_i8_kernel(DepthwiseDesc d, const int8_t* x, const int8_t* w, uint8_t* out,
                                                    uint32_t* err, int64_t total)
{
    constexpr int T = KH * KW;
    constexpr int G = (T + 3) / 4;
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int cg = d.c >> 2;
    const int g = int(idx % cg);
    int64_t r = idx / cg;
    const int owg = (d.ow + PX - 1) / PX;
    const int oxq = int(r % owg);
    r /= owg;
    const int oy = int(r % d.oh);
    const int b = int(r / d.oh);
    const int c0 = 4 * g;

    // Weights [KH][KW][C][1]: words of 4 channels per tap, transposed to 4
    // taps per channel.
    uint32_t wt[G][4];
    int32_t wsum[4] = {0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < G; q++) {
        uint32_t wd[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int t = 4 * q + u;
            wd[u] = t < T ? *reinterpret_cast<const uint32_t*>(w + int64_t(t) * d.c + c0) : 0u;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            wt[q][j] = gather_byte(wd[0], wd[1], wd[2], wd[3], j);
            wsum[j] = __builtin_amdgcn_sdot4(int(wt[q][j]), 0x01010101, wsum[j], false);
        }
    }
    const uint32_t zfill = uint32_t(uint8_t(d.zp_x)) * 0x01010101u;
    const uint32_t tzz = uint32_t(T) * uint32_t(d.zp_x) * uint32_t(d.zp_w);
    int32_t bias[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        bias[j] = d.bias ? d.bias[d.bias_len == 1 ? 0 : c0 + j] : 0;
    uint32_t e = 0;

#pragma unroll
    for (int px = 0; px < PX; px++) {
        const int ox = oxq * PX + px;
        if (ox >= d.ow)
            break;
        const int iy0 = oy * d.sy - d.pt, ix0 = ox * d.sx - d.pl;
        uint32_t acc[4] = {0, 0, 0, 0};
        int32_t xs[4] = {0, 0, 0, 0};
#pragma unroll
        for (int q = 0; q < G; q++) {
            uint32_t xd[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int t = 4 * q + u;
                if (t < T) {
                    const int iy = iy0 + (t / KW) * d.dy, ix = ix0 + (t % KW) * d.dx;
                    xd[u] = (unsigned(iy) < unsigned(d.ih) && unsigned(ix) < unsigned(d.iw))
                                ? *reinterpret_cast<const uint32_t*>(
                                      x + ((int64_t(b) * d.ih + iy) * d.iw + ix) * d.c + c0)
                                : zfill;
                } else {
                    xd[u] = 0u;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t xt = gather_byte(xd[0], xd[1], xd[2], xd[3], j);
                acc[j] = uint32_t(__builtin_amdgcn_sdot4(int(xt), int(wt[q][j]), int(acc[j]), false));
                if (d.zp_w != 0)
                    xs[j] = __builtin_amdgcn_sdot4(int(xt), 0x01010101, xs[j], false);
            }
        }
        const int64_t o = ((int64_t(b) * d.oh + oy) * d.ow + ox) * d.c + c0;
        uint32_t v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            uint32_t a = acc[j] - uint32_t(d.zp_w) * uint32_t(xs[j]) - uint32_t(d.zp_x) * uint32_t(wsum[j]) + tzz +
                         uint32_t(bias[j]);
            if (d.epi == EPI_RESCALE) {
                const int ch = d.rs.per_channel ? c0 + j : 0;
                a = uint32_t(rescale_value(int64_t(int32_t(a)), d.rs.mult[ch], d.rs.shift[ch], d.rs, e));
            }
            v[j] = a;
        }
        if (d.epi == EPI_I32) {
            *reinterpret_cast<uint4*>(out + 4 * o) = uint4{v[0], v[1], v[2], v[3]};
        } else if (d.rs.out_bytes == 1) {
            *reinterpret_cast<uint32_t*>(out + o) =
                (v[0] & 0xFF) | ((v[1] & 0xFF) << 8) | ((v[2] & 0xFF) << 16) | ((v[3] & 0xFF) << 24);
        } else if (d.rs.out_bytes == 2) {
            *reinterpret_cast<uint2*>(out + 2 * o) = uint2{(v[0] & 0xFFFF) | (v[1] << 16), (v[2] & 0xFFFF) | (v[3] << 16)};
        } else {
            *reinterpret_cast<uint4*>(out + 4 * o) = uint4{v[0], v[1], v[2], v[3]};
        }
    }
    report(err, e);
}

// ---------------------------------------------------------------------------
// AVG_POOL2D, src/ops/pool.rs:164-231: padding is excluded from the sum and
// the divisor; integers divide by reciprocal_scale + apply_scale_32
// (src/ops/quant.rs:6-32), floats round every add and the divide.
// ---------------------------------------------------------------------------
__global__ void avg_pool_kernel(PoolDesc d, const void* x, void* out, uint32_t* err, int64_t total)
{
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int c = int(idx % d.c);
    int64_t r = idx / d.c;
    const int ox = int(r % d.ow);
    r /= d.ow;
    const int oy = int(r % d.oh);
    const int b = int(r / d.oh);
    const bool is_int = d.xe == E_I8 || d.xe == E_I16;
    uint32_t acc = 0;
    float facc = 0.0f;
    int32_t count = 0;
    for (int ky = 0; ky < d.kh; ky++) {
        const int y = oy * d.sy - d.pt + ky;
        if (y < 0 || y >= d.ih)
            continue;
        for (int kx = 0; kx < d.kw; kx++) {
            const int xx = ox * d.sx - d.pl + kx;
            if (xx < 0 || xx >= d.iw)
                continue;
            const int64_t i = ((int64_t(b) * d.ih + y) * d.iw + xx) * d.c + c;
            if (is_int)
                acc += uint32_t(int32_t(load_int(x, i, d.xe) - d.in_zp));
            else
                facc = round_fmt(facc + load_float(x, i, d.xe), d.acc_fmt);
            count++;
        }
    }
    if (is_int) {
        // reciprocal_scale(count)
        const uint32_t c1 = uint32_t(count) - 1u;
        const int k = c1 == 0 ? 0 : 32 - __clz(int(c1));
        const int64_t numer = ((int64_t(1) << 30) + 1) << k;
        const int32_t mult = int32_t(numer / count);
        uint32_t e = 0;
        const int32_t v = apply_scale_32(int32_t(acc), mult, 30 + k, false, e);
        report(err, e);
        int64_t o = int64_t(v) + d.out_zp;
        o = o < d.lo ? d.lo : (o > d.hi ? d.hi : o);
        store_int(out, idx, d.xe, o);
    } else {
        const float avg = round_fmt(facc / float(count), d.acc_fmt);
        store_float(out, idx, d.out_fmt, round_fmt(avg, d.out_fmt));
    }
}

// Global average pool over 7x7-style windows of int8 (the head of a
// quantised CNN): 4 channels per thread with word loads.
__global__ void avg_pool_i8_c4_kernel(PoolDesc d, const int8_t* x, int8_t* out, uint32_t* err, int64_t total)
{
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int cg = d.c >> 2;
    const int c0 = 4 * int(idx % cg);
    int64_t r = idx / cg;
    const int ox = int(r % d.ow);
    r /= d.ow;
    const int oy = int(r % d.oh);
    const int b = int(r / d.oh);
    // The in-bounds part of the window (padding positions are excluded from
    // the sum and the count), walked as one flat loop so that many of its
    // loads are in flight at once.
    const int y0 = oy * d.sy - d.pt, x0 = ox * d.sx - d.pl;
    const int ky0 = y0 < 0 ? -y0 : 0, ky1 = d.kh < d.ih - y0 ? d.kh : d.ih - y0;
    const int kx0 = x0 < 0 ? -x0 : 0, kx1 = d.kw < d.iw - x0 ? d.kw : d.iw - x0;
    const int wv = kx1 - kx0;
    const int32_t count = ky1 > ky0 && wv > 0 ? (ky1 - ky0) * wv : 0;
    uint32_t acc[4] = {0, 0, 0, 0};
    if (count > 0) {
        const int8_t* base = x + ((int64_t(b) * d.ih + y0 + ky0) * d.iw + x0 + kx0) * d.c + c0;
        int row = 0, col = 0;
#pragma unroll 16
        for (int t = 0; t < count; t++) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(base + (int64_t(row) * d.iw + col) * d.c);
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[j] += uint32_t(int32_t(int8_t(v >> (8 * j))) - int32_t(d.in_zp));
            if (++col == wv) {
                col = 0;
                row++;
            }
        }
    }
    const uint32_t c1 = uint32_t(count) - 1u;
    const int k = c1 == 0 ? 0 : 32 - __clz(int(c1));
    const int64_t numer = ((int64_t(1) << 30) + 1) << k;
    const int32_t mult = int32_t(numer / count);
    uint32_t e = 0, packed = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int32_t v = apply_scale_32(int32_t(acc[j]), mult, 30 + k, false, e);
        int64_t o = int64_t(v) + d.out_zp;
        o = o < d.lo ? d.lo : (o > d.hi ? d.hi : o);
        packed |= (uint32_t(o) & 0xFFu) << (8 * j);
    }
    report(err, e);
    *reinterpret_cast<uint32_t*>(out + ((int64_t(b) * d.oh + oy) * d.ow + ox) * d.c + c0) = packed;
}

// ---------------------------------------------------------------------------
// RESCALE, src/ops/type_conv.rs:111-191 (per element :174-188).
// ---------------------------------------------------------------------------
__global__ void rescale_kernel(RescaleDev rs, int xe, const void* x, int64_t count, void* out, uint32_t* err)
{
    uint32_t e = 0;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x) {
        const int ch = rs.per_channel ? int(i % rs.channels) : 0;
        const int64_t v = rescale_value(load_int(x, i, xe), rs.mult[ch], rs.shift[ch], rs, e);
        switch (rs.out_bytes) {
        case 1: static_cast<int8_t*>(out)[i] = int8_t(v); break;
        case 2: static_cast<int16_t*>(out)[i] = int16_t(v); break;
        default: static_cast<int32_t*>(out)[i] = int32_t(v); break;
        }
    }
    report(err, e);
}

// int8 -> int8 RESCALE, 4 elements per thread (channels a multiple of 4).
__global__ void rescale_i8_c4_kernel(RescaleDev rs, const int8_t* x, int64_t count4, int8_t* out, uint32_t* err)
{
    uint32_t e = 0;
    for (int64_t q = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; q < count4; q += int64_t(gridDim.x) * blockDim.x) {
        const uint32_t wv = reinterpret_cast<const uint32_t*>(x)[q];
        const int ch0 = rs.per_channel ? int((4 * q) % rs.channels) : 0;
        uint32_t packed = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int ch = rs.per_channel ? ch0 + j : 0;
            const int64_t v = rescale_value(int8_t(wv >> (8 * j)), rs.mult[ch], rs.shift[ch], rs, e);
            packed |= (uint32_t(v) & 0xFFu) << (8 * j);
        }
        reinterpret_cast<uint32_t*>(out)[q] = packed;
    }
    report(err, e);
}

// ---------------------------------------------------------------------------
// CLAMP, src/ops/elementwise.rs:319-343. Floats: nan_max then nan_min
// (src/ops/common.rs:155-177), rounded to the type.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float nan_pick(float a, float b, int ignore)
{
    if (ignore)
        return (a != a) ? b : a;
    return __builtin_nanf("");
}

__global__ void clamp_kernel(int e, const void* x, int64_t count, int64_t ilo, int64_t ihi, float flo, float fhi,
                             int ignore, void* out)
{
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x) {
        if (e == E_I8 || e == E_I16) {
            int64_t v = load_int(x, i, e);
            v = v > ilo ? v : ilo;
            v = v < ihi ? v : ihi;
            store_int(out, i, e, v);
        } else {
            const float v = load_float(x, i, e);
            float m;
            if (v != v)
                m = nan_pick(v, flo, ignore);
            else
                m = v >= flo ? v : flo;
            float r;
            if (m != m)
                r = nan_pick(m, fhi, ignore);
            else
                r = m < fhi ? m : fhi;
            const int fmt = e == E_F16 ? FMT_F16 : (e == E_BF16 ? FMT_BF16 : FMT_F32);
            store_float(out, i, fmt, round_fmt(r, fmt));
        }
    }
}

// ---------------------------------------------------------------------------
// ADD with broadcasting, src/ops/elementwise.rs:395-397 (+ :57-107, :138-145).
// ---------------------------------------------------------------------------
__global__ void add_kernel(int e, BroadcastDesc bd, const void* a, const void* b, void* out, int64_t count)
{
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x) {
        int64_t rem = i, ia = 0, ib = 0;
        for (int dd = bd.rank - 1; dd >= 0; dd--) {
            const int64_t k = rem % bd.out_dims[dd];
            rem /= bd.out_dims[dd];
            ia += k * bd.a_strides[dd];
            ib += k * bd.b_strides[dd];
        }
        if (e == E_I32) {
            static_cast<int32_t*>(out)[i] =
                int32_t(uint32_t(static_cast<const int32_t*>(a)[ia]) + uint32_t(static_cast<const int32_t*>(b)[ib]));
        } else if (e == E_I64) {
            static_cast<int64_t*>(out)[i] =
                int64_t(uint64_t(static_cast<const int64_t*>(a)[ia]) + uint64_t(static_cast<const int64_t*>(b)[ib]));
        } else {
            const int fmt = e == E_F16 ? FMT_F16 : (e == E_BF16 ? FMT_BF16 : FMT_F32);
            const float r = round_fmt(load_float(a, ia, e) + load_float(b, ib, e), fmt);
            store_float(out, i, fmt, r);
        }
    }
}

// RESCALE(a) + RESCALE(b) -> RESCALE, all elementwise with equal shapes.
__global__ void residual_kernel(RescaleDev ra, RescaleDev rb, RescaleDev ro, const int8_t* a, const int8_t* b,
                                int64_t count, int64_t channels, int8_t* out, uint32_t* err)
{
    uint32_t e = 0;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x) {
        const int ch = int(i % channels);
        const int ca = ra.per_channel ? ch : 0, cb = rb.per_channel ? ch : 0, co = ro.per_channel ? ch : 0;
        const int32_t va = int32_t(rescale_value(a[i], ra.mult[ca], ra.shift[ca], ra, e));
        const int32_t vb = int32_t(rescale_value(b[i], rb.mult[cb], rb.shift[cb], rb, e));
        const int32_t s = int32_t(uint32_t(va) + uint32_t(vb));
        out[i] = int8_t(rescale_value(s, ro.mult[co], ro.shift[co], ro, e));
    }
    report(err, e);
}

__global__ void residual_c4_kernel(RescaleDev ra, RescaleDev rb, RescaleDev ro, const int8_t* a, const int8_t* b,
                                   int64_t count4, int64_t channels, int8_t* out, uint32_t* err)
{
    uint32_t e = 0;
    for (int64_t q = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; q < count4; q += int64_t(gridDim.x) * blockDim.x) {
        const uint32_t wa = reinterpret_cast<const uint32_t*>(a)[q];
        const uint32_t wb = reinterpret_cast<const uint32_t*>(b)[q];
        const int ch0 = int((4 * q) % channels);
        uint32_t packed = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int ch = ch0 + j;
            const int ca = ra.per_channel ? ch : 0, cb = rb.per_channel ? ch : 0, co = ro.per_channel ? ch : 0;
            const int32_t va = int32_t(rescale_value(int8_t(wa >> (8 * j)), ra.mult[ca], ra.shift[ca], ra, e));
            const int32_t vb = int32_t(rescale_value(int8_t(wb >> (8 * j)), rb.mult[cb], rb.shift[cb], rb, e));
            const int32_t s = int32_t(uint32_t(va) + uint32_t(vb));
            packed |= (uint32_t(rescale_value(s, ro.mult[co], ro.shift[co], ro, e)) & 0xFFu) << (8 * j);
        }
        reinterpret_cast<uint32_t*>(out)[q] = packed;
    }
    report(err, e);
}

// Residual block with every REQUIRE settled on the host (see
// residual_fast_ok): a thread owns 4 consecutive channels of the output and
// walks pixels, with the three RESCALEs' multipliers, shifts and rounding
// constants for those channels in registers. Per element:
//   va = apply_scale_32(a - za), vb = apply_scale_32(b - zb)     (int8 -> int32)
//   y  = clamp(apply_scale_32(va + vb (mod 2^32)) + zo)          (int32 -> int8)
// with apply_scale_32 (src/ops/quant.rs:17-32) as one 64-bit multiply-add of
// the sign-selected rounding constant (the output zero point folded into the
// final one) and an arithmetic shift.
struct ResChan {
    int32_t m, s;
    int64_t rp, rn;
};

__device__ __forceinline__ ResChan res_chan(const RescaleDev& r, int c, int64_t zp)
{
    const int ch = r.per_channel ? c : 0;
    ResChan q;
    q.m = r.mult[ch];
    q.s = r.shift[ch];
    const int64_t half = int64_t(1) << (q.s - 1);
    const int64_t d = (r.rounding == 3 && q.s > 31) ? (int64_t(1) << 30) : 0;
    const int64_t z = zp * (int64_t(1) << q.s);
    q.rp = half + d + z;
    q.rn = half - d + z;
    return q;
}

__device__ __forceinline__ int32_t res_scale(int32_t x, const ResChan& q)
{
    return int32_t((int64_t(x) * q.m + (x >= 0 ? q.rp : q.rn)) >> q.s);
}

__global__ void __launch_bounds__(256) residual_fast_kernel(RescaleDev ra, RescaleDev rb, RescaleDev ro,
                                                            const int8_t* a, const int8_t* b, int64_t pixels,
                                                            int32_t channels, int32_t ppb, int8_t* out,
                                                            uint32_t* err)
{
    const int tpp = channels >> 2;  // threads per pixel
    const int t = threadIdx.x;
    if (t >= tpp * ppb)
        return;
    const int cq = t % tpp;
    const int c0 = 4 * cq;
    ResChan qa[4], qb[4], qo[4];
    int32_t lo[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        qa[i] = res_chan(ra, c0 + i, 0);
        qb[i] = res_chan(rb, c0 + i, 0);
        qo[i] = res_chan(ro, c0 + i, ro.out_zp);
        lo[i] = qo[i].s - 1 < 31 ? -(int32_t(1) << (qo[i].s - 1)) : INT32_MIN;
    }
    const int32_t za = int32_t(ra.in_zp), zb = int32_t(rb.in_zp);
    const int32_t clo = int32_t(ro.has_clamp ? (ro.clamp_lo > ro.lo ? ro.clamp_lo : ro.lo) : ro.lo);
    const int32_t chi = int32_t(ro.has_clamp ? (ro.clamp_hi < ro.hi ? ro.clamp_hi : ro.hi) : ro.hi);
    bool bad = false;
    const uint32_t* a4 = reinterpret_cast<const uint32_t*>(a);
    const uint32_t* b4 = reinterpret_cast<const uint32_t*>(b);
    uint32_t* o4 = reinterpret_cast<uint32_t*>(out);
#pragma unroll 2
    for (int64_t p = int64_t(blockIdx.x) * ppb + t / tpp; p < pixels; p += int64_t(gridDim.x) * ppb) {
        const int64_t q = p * tpp + cq;
        const uint32_t wa = a4[q], wb = b4[q];
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int32_t va = res_scale(int32_t(int8_t(wa >> (8 * i))) - za, qa[i]);
            const int32_t vb = res_scale(int32_t(int8_t(wb >> (8 * i))) - zb, qb[i]);
            const int32_t sum = int32_t(uint32_t(va) + uint32_t(vb));
            bad |= sum < lo[i] || sum > ~lo[i];
            int32_t r = res_scale(sum, qo[i]);
            r = r < clo ? clo : (r > chi ? chi : r);
            packed |= (uint32_t(r) & 0xFFu) << (8 * i);
        }
        o4[q] = packed;
    }
    if (bad)
        atomicOr(err, DERR_SCALE_RANGE);
}

// ---------------------------------------------------------------------------
// TRANSPOSE: output element i reads input at sum(index_d * stride_perm[d]).
// ---------------------------------------------------------------------------
struct TransposeArgs {
    int32_t rank;
    int64_t dims[6];
    int64_t strides[6];
};

__global__ void transpose_kernel(const uint8_t* x, uint8_t* out, int esize, TransposeArgs t, int64_t count)
{
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x) {
        int64_t rem = i, src = 0;
        for (int dd = t.rank - 1; dd >= 0; dd--) {
            const int64_t k = rem % t.dims[dd];
            rem /= t.dims[dd];
            src += k * t.strides[dd];
        }
        for (int b = 0; b < esize; b++)
            out[i * esize + b] = x[src * esize + b];
    }
}

unsigned grid_for(int64_t n)
{
    const int64_t b = (n + 255) / 256;
    return static_cast<unsigned>(b < 65536 ? (b < 1 ? 1 : b) : 65536);
}


// MAX_POOL2D (src/ops/pool.rs:233-286): one output per thread; the window's
// in-bounds positions in (ky, kx) order (for_each_window, :77-104).
// Integers fold max from the type's minimum; floats fold nan_max
// (src/ops/common.rs:155-177: ties keep the running value, NaN handled per
// mode) from the type's lowest value, or from NaN under IGNORE.
__global__ void max_pool_kernel(PoolDesc d, bool ignore, float lowest, const void* x, void* out, int64_t total)
{
    const int64_t idx = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= total)
        return;
    const int c = int(idx % d.c);
    int64_t r = idx / d.c;
    const int ox = int(r % d.ow);
    r /= d.ow;
    const int oy = int(r % d.oh);
    const int b = int(r / d.oh);
    const int iy = oy * d.sy - d.pt, ix = ox * d.sx - d.pl;
    const bool is_int = d.xe == E_I8 || d.xe == E_I16;
    int64_t mi = d.xe == E_I8 ? -128 : -32768;
    float mf = ignore ? __builtin_nanf("") : lowest;
    for (int ky = 0; ky < d.kh; ky++) {
        const int y = iy + ky;
        if (y < 0 || y >= d.ih)
            continue;
        for (int kx = 0; kx < d.kw; kx++) {
            const int xx = ix + kx;
            if (xx < 0 || xx >= d.iw)
                continue;
            const int64_t i = ((int64_t(b) * d.ih + y) * d.iw + xx) * d.c + c;
            if (is_int) {
                const int64_t v = load_int(x, i, d.xe);
                mi = v > mi ? v : mi;
            } else {
                const float v = load_float(x, i, d.xe);
                if (__builtin_isnan(mf) || __builtin_isnan(v))
                    mf = ignore ? (__builtin_isnan(mf) ? v : mf) : __builtin_nanf("");
                else
                    mf = mf >= v ? mf : v;
            }
        }
    }
    if (is_int)
        store_int(out, idx, d.xe, mi);
    else
        store_float(out, idx, d.out_fmt, mf);
}

// CAST (src/ops/type_conv.rs:45-80), one element per thread.
__global__ void cast_kernel(CastDesc d, const void* x, int64_t count, void* out)
{
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count)
        return;
    if (!d.from_float) {
        const int64_t v = load_int(x, i, d.from);  // BOOL reads as 0 / 1
        if (d.to_bool)
            store_int(out, i, E_U8, v != 0 ? 1 : 0);
        else if (d.to_float)
            store_float(out, i, d.to_fmt, float(v));  // through FP32, then to the format
        else
            store_int(out, i, d.to, v);  // wraps (int_data)
        return;
    }
    const float v = load_float(x, i, d.from);
    if (d.to_bool) {
        store_int(out, i, E_U8, v != 0.0f ? 1 : 0);
    } else if (d.to_float) {
        store_float(out, i, d.to_fmt, v);
    } else {
        // float_to_int (:34-43): saturate at the bounds as rounded to the
        // input's precision, else round half to even; NaN becomes 0.
        int64_t q;
        if (v >= d.hi_bound)
            q = d.hi;
        else if (v <= d.lo_bound)
            q = d.lo;
        else if (__builtin_isnan(v))
            q = 0;
        else
            q = int64_t(__builtin_rintf(v));
        store_int(out, i, d.to, q);
    }
}


// int16 values as two int8 halves for the int8 MFMA kernels: x = 256 hi +
// lo with hi = x >> 8 (arithmetic) and lo = x & 255, stored as lo - 128 so
// that it fits int8 (a kernel input zero point of -128 gives lo back).
__global__ void split_i16_kernel(const int16_t* x, int64_t count, int8_t* hi, int8_t* lo)
{
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count)
        return;
    const int32_t v = x[i];
    hi[i] = int8_t(v >> 8);
    lo[i] = int8_t((v & 255) - 128);
}

// The same, 8 values per thread (16-byte loads, 8-byte stores) for 16-byte
// aligned x, 8-byte aligned halves and a count that is a multiple of 8.
__global__ void split_i16_x8_kernel(const uint4* x, int64_t count8, uint2* hi, uint2* lo)
{
    for (int64_t q = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; q < count8; q += int64_t(gridDim.x) * blockDim.x) {
        const uint4 v = x[q];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t h[2], l[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            // high bytes of the four int16 values in words 2k, 2k + 1 (v_perm_b32:
            // selector bytes 0-3 pick the second operand, 4-7 the first); low
            // bytes likewise, then each offset by -128 (bit 7 flipped).
            h[k] = __builtin_amdgcn_perm(w[2 * k + 1], w[2 * k], 0x07050301u);
            l[k] = __builtin_amdgcn_perm(w[2 * k + 1], w[2 * k], 0x06040200u) ^ 0x80808080u;
        }
        hi[q] = uint2{h[0], h[1]};
        lo[q] = uint2{l[0], l[1]};
    }
}

// INT48 result of products of int16 operands assembled from int32 partial
// sums of their int8 halves: out = clamp48(sum_k coef[k] part[k] + bias),
// in int64 (the reference's AccI64 and its final clamp, src/ops/conv.rs:
// 465-473, src/ops/matmul.rs:150-153).
struct I48Parts {
    const int32_t* part[4];
    int64_t coef[4];
    int32_t nparts;
    const int64_t* bias;  // [bias_len] or null
    int32_t bias_len;
    int32_t channels;     // bias index = i % channels when bias_len > 1
};

__global__ void combine_i48_kernel(I48Parts p, int64_t count, int64_t* out)
{
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count)
        return;
    int64_t v = 0;
    for (int k = 0; k < p.nparts; k++)
        v += p.coef[k] * int64_t(p.part[k][i]);
    if (p.bias)
        v += p.bias[p.bias_len == 1 ? 0 : i % p.channels];
    const int64_t lo = -(int64_t(1) << 47), hi = (int64_t(1) << 47) - 1;
    out[i] = v < lo ? lo : (v > hi ? hi : v);
}

// The INT48 combine followed by the RESCALE that reads it: each combined,
// clamped value goes straight into the RESCALE (eval_rescale's per-element
// steps, rescale_value), with no int64 tensor in between.
// Elements below 2^31 (host-checked); the channel of element i, i mod
// channels, by a multiply-high division.
__global__ void combine_i48_rescale_kernel(I48Parts p, RescaleDev rs, int32_t count, FastDiv div_c, void* out,
                                           uint32_t* err)
{
    uint32_t e = 0;
    const int64_t lo = -(int64_t(1) << 47), hi = (int64_t(1) << 47) - 1;
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += int64_t(gridDim.x) * blockDim.x) {
        const int32_t c = int32_t(i) - int32_t(fdiv(uint32_t(i), div_c)) * p.channels;
        int64_t v = 0;
        for (int k = 0; k < p.nparts; k++)
            v += p.coef[k] * int64_t(p.part[k][i]);
        if (p.bias)
            v += p.bias[p.bias_len == 1 ? 0 : c];
        v = v < lo ? lo : (v > hi ? hi : v);
        const int ch = rs.per_channel ? c : 0;
        const int64_t r = rescale_value(v, rs.mult[ch], rs.shift[ch], rs, e);
        switch (rs.out_bytes) {
        case 1: static_cast<int8_t*>(out)[i] = int8_t(r); break;
        case 2: static_cast<int16_t*>(out)[i] = int16_t(r); break;
        default: static_cast<int32_t*>(out)[i] = int32_t(r); break;
        }
    }
    report(err, e);
}

}  // namespace

// The residual kernel without per-element checks applies when every REQUIRE
// of the three RESCALEs is settled by the parameters: int8 -> int32 with
// SINGLE/DOUBLE rounding and shifts >= 9 (|a - za| <= 255 < 2^(s-1), and the
// scaled value fits int32), int32 -> int8 with SINGLE/DOUBLE rounding and an
// output zero point that folds into the rounding constant; 4-byte aligned
// rows of channels % 4 == 0 values, at most 1024 channels.
static bool residual_fast_ok(const RescaleDev& ra, const RescaleDev& rb, const RescaleDev& ro, int64_t count,
                      int64_t channels, const void* a, const void* b, const void* out)
{
    auto in_ok = [channels](const RescaleDev& r) {
        return r.scale32 && (r.rounding == 1 || r.rounding == 3) && r.in_bits == 8 && !r.in_unsigned &&
               r.out_bytes == 4 && r.out_zp == 0 && !r.has_clamp && r.min_shift >= 9 &&
               (!r.per_channel || r.channels == channels);
    };
    const int64_t zp = ro.out_zp < 0 ? -ro.out_zp : ro.out_zp;
    const bool fold = zp == 0 || (ro.max_shift <= 60 && zp <= (int64_t(1) << (60 - ro.max_shift)));
    const bool o_ok = ro.scale32 && (ro.rounding == 1 || ro.rounding == 3) && ro.in_bits == 32 && !ro.in_unsigned &&
                      ro.in_zp == 0 && ro.out_bytes == 1 && fold && (!ro.per_channel || ro.channels == channels);
    const bool aligned = (reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                          reinterpret_cast<uintptr_t>(out)) % 4 == 0;
    return in_ok(ra) && in_ok(rb) && o_ok && aligned && channels % 4 == 0 && channels >= 4 && channels <= 1024 &&
           count % channels == 0;
}

bool depthwise_i8_supported(int kh, int kw, int c)
{
    const bool taps = (kh == 3 && kw == 3) || (kh == 1 && kw == 1) || (kh == 1 && kw == 3) || (kh == 3 && kw == 1) ||
                      (kh == 2 && kw == 2);
    return taps && c % 4 == 0;
}

void depthwise_i8(const DepthwiseDesc& d, const int8_t* x, const int8_t* w, void* out, uint32_t* err,
                  hipStream_t stream)
{
    constexpr int PX = 4;
    const int64_t total = int64_t(d.n) * d.oh * ((d.ow + PX - 1) / PX) * (d.c / 4);
    if (total <= 0 || !depthwise_i8_supported(d.kh, d.kw, d.c))
        return;
    const dim3 grid(blocks_for(total, 256));
    uint8_t* o = static_cast<uint8_t*>(out);
    if (d.kh == 3 && d.kw == 3)
        hipLaunchKernelGGL((dw_i8_kernel<3, 3, PX>), grid, dim3(256), 0, stream, d, x, w, o, err, total);
    else if (d.kh == 1 && d.kw == 1)
        hipLaunchKernelGGL((dw_i8_kernel<1, 1, PX>), grid, dim3(256), 0, stream, d, x, w, o, err, total);
    else if (d.kh == 1 && d.kw == 3)
        hipLaunchKernelGGL((dw_i8_kernel<1, 3, PX>), grid, dim3(256), 0, stream, d, x, w, o, err, total);
    else if (d.kh == 3 && d.kw == 1)
        hipLaunchKernelGGL((dw_i8_kernel<3, 1, PX>), grid, dim3(256), 0, stream, d, x, w, o, err, total);
    else
        hipLaunchKernelGGL((dw_i8_kernel<2, 2, PX>), grid, dim3(256), 0, stream, d, x, w, o, err, total);
}

void avg_pool2d(const PoolDesc& d, const void* x, void* out, uint32_t* err, hipStream_t stream)
{
    const int64_t total = int64_t(d.n) * d.oh * d.ow * d.c;
    if (total <= 0)
        return;
    if (d.xe == E_I8 && d.c % 4 == 0) {
        const int64_t t4 = total / 4;
        hipLaunchKernelGGL(avg_pool_i8_c4_kernel, dim3(blocks_for(t4, 256)), dim3(256), 0, stream, d,
                           static_cast<const int8_t*>(x), static_cast<int8_t*>(out), err, t4);
    } else {
        hipLaunchKernelGGL(avg_pool_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, stream, d, x, out, err, total);
    }
}

void split_i16(const int16_t* x, int64_t count, int8_t* hi, int8_t* lo, hipStream_t stream)
{
    if (count <= 0)
        return;
    const bool x8 = count % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                    (reinterpret_cast<uintptr_t>(hi) | reinterpret_cast<uintptr_t>(lo)) % 8 == 0;
    if (x8)
        hipLaunchKernelGGL(split_i16_x8_kernel, dim3(grid_for(count / 8)), dim3(256), 0, stream,
                           reinterpret_cast<const uint4*>(x), count / 8, reinterpret_cast<uint2*>(hi),
                           reinterpret_cast<uint2*>(lo));
    else
        hipLaunchKernelGGL(split_i16_kernel, dim3(blocks_for(count, 256)), dim3(256), 0, stream, x, count, hi, lo);
}

void combine_i48(const int32_t* const* parts, const int64_t* coef, int nparts, const int64_t* bias, int32_t bias_len,
                 int32_t channels, int64_t count, int64_t* out, hipStream_t stream)
{
    I48Parts p{};
    p.nparts = nparts;
    for (int k = 0; k < nparts; k++) {
        p.part[k] = parts[k];
        p.coef[k] = coef[k];
    }
    p.bias = bias;
    p.bias_len = bias_len;
    p.channels = channels;
    if (count > 0)
        hipLaunchKernelGGL(combine_i48_kernel, dim3(blocks_for(count, 256)), dim3(256), 0, stream, p, count, out);
}

void combine_i48_rescale(const int32_t* const* parts, const int64_t* coef, int nparts, const int64_t* bias,
                         int32_t bias_len, int32_t channels, int64_t count, const RescaleDev& rs, void* out,
                         uint32_t* err, hipStream_t stream)
{
    I48Parts p{};
    p.nparts = nparts;
    for (int k = 0; k < nparts; k++) {
        p.part[k] = parts[k];
        p.coef[k] = coef[k];
    }
    p.bias = bias;
    p.bias_len = bias_len;
    p.channels = channels;
    if (count >= (int64_t(1) << 31) || channels < 1 || (rs.per_channel && rs.channels != channels))
        throw std::runtime_error("combine_i48_rescale: unsupported size or channel count");
    if (count > 0)
        hipLaunchKernelGGL(combine_i48_rescale_kernel, dim3(grid_for(count)), dim3(256), 0, stream, p, rs,
                           int32_t(count), FastDiv(uint32_t(channels)), out, err);
}

void max_pool2d(const PoolDesc& d, bool ignore, float lowest, const void* x, void* out, hipStream_t stream)
{
    const int64_t total = int64_t(d.n) * d.oh * d.ow * d.c;
    if (total > 0)
        hipLaunchKernelGGL(max_pool_kernel, dim3(blocks_for(total, 256)), dim3(256), 0, stream, d, ignore, lowest, x,
                           out, total);
}

void cast(const CastDesc& d, const void* x, int64_t count, void* out, hipStream_t stream)
{
    if (count > 0)
        hipLaunchKernelGGL(cast_kernel, dim3(blocks_for(count, 256)), dim3(256), 0, stream, d, x, count, out);
}

void rescale(const RescaleDev& rs, ElemCode xe, const void* x, int64_t count, void* out, uint32_t* err,
             hipStream_t stream)
{
    if (count <= 0)
        return;
    if (xe == E_I8 && rs.out_bytes == 1 && count % 4 == 0 && (!rs.per_channel || rs.channels % 4 == 0)) {
        hipLaunchKernelGGL(rescale_i8_c4_kernel, dim3(grid_for(count / 4)), dim3(256), 0, stream, rs,
                           static_cast<const int8_t*>(x), count / 4, static_cast<int8_t*>(out), err);
        return;
    }
    hipLaunchKernelGGL(rescale_kernel, dim3(grid_for(count)), dim3(256), 0, stream, rs, int(xe), x, count, out, err);
}

void clamp(ElemCode e, const void* x, int64_t count, int64_t ilo, int64_t ihi, float flo, float fhi, int nan_ignore,
           void* out, hipStream_t stream)
{
    if (count > 0)
        hipLaunchKernelGGL(clamp_kernel, dim3(grid_for(count)), dim3(256), 0, stream, int(e), x, count, ilo, ihi, flo,
                           fhi, nan_ignore, out);
}

void add(ElemCode e, const BroadcastDesc& bd, const void* a, const void* b, void* out, int64_t count,
         hipStream_t stream)
{
    if (count > 0)
        hipLaunchKernelGGL(add_kernel, dim3(grid_for(count)), dim3(256), 0, stream, int(e), bd, a, b, out, count);
}

void residual_add_i8(const RescaleDev& ra, const RescaleDev& rb, const RescaleDev& ro, const int8_t* a,
                     const int8_t* b, int64_t count, int64_t channels, void* out, uint32_t* err,
                     hipStream_t stream)
{
    if (count <= 0)
        return;
    if (residual_fast_ok(ra, rb, ro, count, channels, a, b, out)) {
        const int tpp = int(channels / 4);
        const int ppb = 256 / tpp;
        const int64_t pixels = count / channels;
        // Two workgroups per CU walk the pixels: each thread's setup (the
        // three RESCALEs' parameters of its four channels) then serves many
        // pixels instead of one or two.
        const int64_t blocks = std::min<int64_t>((pixels + ppb - 1) / ppb, 2 * int64_t(cu_count()));
        hipLaunchKernelGGL(residual_fast_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                           stream, ra, rb, ro, a, b, pixels, int32_t(channels), ppb, static_cast<int8_t*>(out), err);
        return;
    }
    if (count % 4 == 0 && channels % 4 == 0)
        hipLaunchKernelGGL(residual_c4_kernel, dim3(grid_for(count / 4)), dim3(256), 0, stream, ra, rb, ro, a, b,
                           count / 4, channels, static_cast<int8_t*>(out), err);
    else
        hipLaunchKernelGGL(residual_kernel, dim3(grid_for(count)), dim3(256), 0, stream, ra, rb, ro, a, b, count,
                           channels, static_cast<int8_t*>(out), err);
}

void transpose(const void* x, void* out, int32_t esize, int32_t rank, const int64_t* out_dims,
               const int64_t* in_strides_permuted, int64_t count, hipStream_t stream)
{
    if (count <= 0)
        return;
    TransposeArgs t{};
    t.rank = rank;
    for (int i = 0; i < rank; i++) {
        t.dims[i] = out_dims[i];
        t.strides[i] = in_strides_permuted[i];
    }
    hipLaunchKernelGGL(transpose_kernel, dim3(grid_for(count)), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(x), static_cast<uint8_t*>(out), esize, t, count);
}

}  // namespace kern
}  // namespace tosa
