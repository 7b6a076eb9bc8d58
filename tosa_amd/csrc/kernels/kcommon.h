// Device helpers shared by the gfx950 kernels: the reference's fixed-point
// scaling (src/ops/quant.rs, src/ops/type_conv.rs:86-188), float rounding to
// the TOSA storage formats, and typed element loads.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "../device.h"
#include "../kernels.h"

namespace tosa {
namespace kern {

// Median of three (v_med3_i32): clamp of v to [lo, hi] when lo <= hi.
__device__ __forceinline__ int32_t med3_i32(int32_t v, int32_t lo, int32_t hi)
{
    int32_t r;
    asm("v_med3_i32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "v"(lo), "v"(hi));
    return r;
}

// Four values' low bytes packed into one word: two byte permutes (v_perm_b32
// selector bytes 0-3 pick the second operand, 4-7 the first, 0x0c gives 0)
// and an OR.
__device__ __forceinline__ uint32_t pack4_u8(int32_t v0, int32_t v1, int32_t v2, int32_t v3)
{
    const uint32_t lo = __builtin_amdgcn_perm(uint32_t(v1), uint32_t(v0), 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm(uint32_t(v3), uint32_t(v2), 0x04000c0cu);
    return lo | hi;
}

// q = n / d for n < 2^31: (mulhi(n, m) + n) >> s.
__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) { return (__umulhi(n, f.m) + n) >> f.s; }

// apply_scale_32 (src/ops/quant.rs:17-32) without the parameter checks,
// which the host has done for every channel.
__device__ __forceinline__ int32_t apply_scale_32(int32_t value, int32_t mult, int32_t shift, bool dbl,
                                                  uint32_t& err)
{
    const int64_t half = int64_t(1) << (shift - 1);
    const int64_t v = value;
    if (shift <= 32 && (v < -half || v >= half)) {
        err |= DERR_SCALE_RANGE;
        return 0;
    }
    int64_t round = half;
    if (dbl && shift > 31)
        round += v >= 0 ? (int64_t(1) << 30) : -(int64_t(1) << 30);
    const int64_t r = (v * mult + round) >> shift;
    if (r < INT32_MIN || r > INT32_MAX) {
        err |= DERR_SCALE_RESULT;
        return 0;
    }
    return static_cast<int32_t>(r);
}

// apply_scale_16 (src/ops/type_conv.rs:86-92) without the parameter checks.
__device__ __forceinline__ int32_t apply_scale_16(int64_t value, int32_t mult, int32_t shift, uint32_t& err)
{
    const int64_t r = static_cast<int64_t>(static_cast<uint64_t>(value) * static_cast<uint64_t>(int64_t(mult)) +
                                           (uint64_t(1) << (shift - 1))) >>
                      shift;
    if (r < INT32_MIN || r > INT32_MAX) {
        err |= DERR_SCALE_RESULT;
        return 0;
    }
    return static_cast<int32_t>(r);
}

__device__ __forceinline__ int32_t sat_f32_to_i32(float f)
{
    if (f != f)
        return 0;
    if (f >= 2147483648.0f)
        return INT32_MAX;
    if (f < -2147483648.0f)
        return INT32_MIN;
    return static_cast<int32_t>(f);
}

// One RESCALE element (src/ops/type_conv.rs:174-188) plus an optional CLAMP
// of the stored value; `v` is the input element sign-extended to int64.
__device__ __forceinline__ int64_t rescale_value(int64_t v, int32_t m, int32_t s, const RescaleDev& rs, uint32_t& err)
{
    if (rs.in_unsigned)
        v &= static_cast<int64_t>((uint64_t(1) << rs.in_bits) - 1);
    const int64_t x = v - rs.in_zp;
    int32_t scaled;
    if (rs.rounding == 2) {
#pragma clang fp contract(off)
        const float p = static_cast<float>(x) * static_cast<float>(m);
        scaled = sat_f32_to_i32(rintf(p * ldexpf(1.0f, -s)));
    } else if (rs.scale32) {
        scaled = apply_scale_32(static_cast<int32_t>(x), m, s, rs.rounding == 3, err);
    } else {
        scaled = apply_scale_16(x, static_cast<int16_t>(m), s, err);
    }
    int64_t r = static_cast<int64_t>(scaled) + rs.out_zp;
    if (r < INT32_MIN || r > INT32_MAX)
        err |= DERR_RESCALE_I32;
    r = r < rs.lo ? rs.lo : (r > rs.hi ? rs.hi : r);
    if (rs.has_clamp) {
        // CLAMP reads the stored value: wrap to the output width first.
        const int sh = 64 - 8 * rs.out_bytes;
        r = static_cast<int64_t>(static_cast<uint64_t>(r) << sh) >> sh;
        r = r < rs.clamp_lo ? rs.clamp_lo : (r > rs.clamp_hi ? rs.clamp_hi : r);
    }
    return r;
}

// ---------------------------------------------------------------------------
// Float formats
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b)
{
    return __builtin_bit_cast(float, static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// FP8 (OCP E4M3FN / E5M2) decode and round-to-nearest-even encode with the
// reference's overflow rule: E4M3 overflows to NaN, E5M2 to infinity
// (src/float8.rs:1-10). Computed in double, where every scaling by a power of
// two is exact.
__device__ __forceinline__ float fp8_to_f32(uint8_t b, bool e4m3)
{
    const int mb = e4m3 ? 3 : 2, bias = e4m3 ? 7 : 15, maxe = e4m3 ? 15 : 31;
    const int e = (b >> mb) & maxe, m = b & ((1 << mb) - 1);
    const float sign = (b & 0x80) ? -1.0f : 1.0f;
    if (e4m3 ? (e == 15 && m == 7) : (e == 31 && m != 0))
        return __builtin_nanf("");
    if (!e4m3 && e == 31)
        return sign * __builtin_inff();
    const double mag = e == 0 ? ldexp(static_cast<double>(m), 1 - bias - mb)
                              : ldexp(static_cast<double>((1 << mb) + m), e - bias - mb);
    return static_cast<float>(sign * mag);
}

__device__ __forceinline__ uint8_t f32_to_fp8(float x, bool e4m3)
{
    const int mb = e4m3 ? 3 : 2, bias = e4m3 ? 7 : 15, maxe = e4m3 ? 15 : 31;
    const uint32_t mmask = (1u << mb) - 1;
    const uint8_t nan = static_cast<uint8_t>((maxe << mb) | mmask);
    if (x != x)
        return nan;
    const uint8_t sign = (__builtin_bit_cast(uint32_t, x) >> 31) ? 0x80 : 0;
    const uint8_t overflow = e4m3 ? static_cast<uint8_t>(sign | nan) : static_cast<uint8_t>(sign | (maxe << mb));
    const double a = fabs(static_cast<double>(x));
    if (a == __builtin_inf())
        return overflow;
    if (a == 0.0)
        return sign;
    const int min_normal = 1 - bias;
    int e = ilogb(a);
    uint32_t ef, man;
    if (e < min_normal) {
        const uint32_t q = static_cast<uint32_t>(rint(ldexp(a, mb - min_normal)));
        ef = q >> mb;
        man = q & mmask;
    } else {
        uint32_t q = static_cast<uint32_t>(rint(ldexp(a, mb - e)));
        if (q == (2u << mb)) {
            e += 1;
            q = 1u << mb;
        }
        ef = static_cast<uint32_t>(e + bias);
        man = q & mmask;
    }
    const bool exceeded = e4m3 ? (ef > 15u || (ef == 15u && man == mmask)) : (ef >= 31u);
    if (exceeded)
        return overflow;
    return static_cast<uint8_t>(sign | (ef << mb) | man);
}

// round_to (src/ops/common.rs:100-108)
__device__ __forceinline__ float round_fmt(float x, int fmt)
{
    switch (fmt) {
    case FMT_F16: return f16_bits_to_f32(f32_to_f16_bits(x));
    case FMT_BF16: return bf16_bits_to_f32(f32_to_bf16_bits(x));
    case FMT_FP8E4M3: return fp8_to_f32(f32_to_fp8(x, true), true);
    case FMT_FP8E5M2: return fp8_to_f32(f32_to_fp8(x, false), false);
    default: return x;
    }
}

// round_to restricted to the MFMA epilogue's formats (F32, F16, BF16).
__device__ __forceinline__ float round_fmt16(float x, int fmt)
{
    if (fmt == FMT_F16)
        return f16_bits_to_f32(f32_to_f16_bits(x));
    if (fmt == FMT_BF16)
        return bf16_bits_to_f32(f32_to_bf16_bits(x));
    return x;
}

// ---------------------------------------------------------------------------
// Typed element access
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t load_int(const void* p, int64_t i, int e)
{
    switch (e) {
    case E_I8: return static_cast<const int8_t*>(p)[i];
    case E_U8: return static_cast<const uint8_t*>(p)[i];
    case E_I16: return static_cast<const int16_t*>(p)[i];
    case E_I32: return static_cast<const int32_t*>(p)[i];
    default: return static_cast<const int64_t*>(p)[i];
    }
}

__device__ __forceinline__ float load_float(const void* p, int64_t i, int e)
{
    switch (e) {
    case E_F16: return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    case E_BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    case E_FP8E4M3: return fp8_to_f32(static_cast<const uint8_t*>(p)[i], true);
    case E_FP8E5M2: return fp8_to_f32(static_cast<const uint8_t*>(p)[i], false);
    default: return static_cast<const float*>(p)[i];
    }
}

__device__ __forceinline__ void store_int(void* p, int64_t i, int e, int64_t v)
{
    switch (e) {
    case E_I8:
    case E_U8: static_cast<int8_t*>(p)[i] = static_cast<int8_t>(v); break;
    case E_I16: static_cast<int16_t*>(p)[i] = static_cast<int16_t>(v); break;
    case E_I32: static_cast<int32_t*>(p)[i] = static_cast<int32_t>(v); break;
    default: static_cast<int64_t*>(p)[i] = v; break;
    }
}

// Store a float already rounded to `fmt` in that format's storage.
__device__ __forceinline__ void store_float(void* p, int64_t i, int fmt, float v)
{
    switch (fmt) {
    case FMT_F16: static_cast<uint16_t*>(p)[i] = f32_to_f16_bits(v); break;
    case FMT_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v); break;
    case FMT_FP8E4M3: static_cast<uint8_t*>(p)[i] = f32_to_fp8(v, true); break;
    case FMT_FP8E5M2: static_cast<uint8_t*>(p)[i] = f32_to_fp8(v, false); break;
    default: static_cast<float*>(p)[i] = v; break;
    }
}

__device__ __forceinline__ void report(uint32_t* err, uint32_t bits)
{
    if (bits)
        atomicOr(err, bits);
}

inline unsigned blocks_for(int64_t n, int threads) { return static_cast<unsigned>((n + threads - 1) / threads); }

}  // namespace kern
}  // namespace tosa
