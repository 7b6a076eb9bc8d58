/*
 * CPU oracle for the TOSA hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference interpreter's arithmetic for
 * CONV2D, DEPTHWISE_CONV2D, MATMUL, AVG_POOL2D and RESCALE (emmet-horgan/tosa,
 * `tosa-interp`, Rust). It follows the reference's loop order and rounding
 * step by step so that float results are bit-identical to a sequential
 * evaluation; integer results are order-independent mod 2^32.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker / CPU baseline. The product
 * (tosa_amd/) never links or calls it.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; x86-64 SSE arithmetic,
 * so every float operation is a single IEEE-754 binary32 operation, as in
 * Rust, which never contracts a*b+c into an FMA).
 *
 * Operands arrive widened: integers as int64 (the reference's `int_values`,
 * src/ops/common.rs:63-71), floats as f32 holding exactly representable
 * values of their TOSA type (`float_values`, src/ops/common.rs:75-84).
 *
 * Parity status of each function is stated in its comment; every function
 * here is pinned by the golden fixtures (tests/test_oracle.py) and, for the
 * integer paths, by an independent numpy brute force.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_OK 0
#define ORC_ERR (-1)

/* Float formats used for rounding (subset of src/ir.rs:5-27). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2, ORC_FP8E4M3 = 3, ORC_FP8E5M2 = 4 };

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---------------------------------------------------------------------------
 * IEEE binary16 / bfloat16, round to nearest even. The reference uses the
 * `half` crate 2.7.1 (`f16::from_f32`, `bf16::from_f32`; call sites
 * src/ops/common.rs:91-92,102-103). Restated from IEEE-754 RNE; pinned by the
 * f16/bf16 fixtures and by an exhaustive comparison with numpy's float16.
 * ------------------------------------------------------------------------- */
uint16_t orc_f16_bits(float f)
{
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff)
        return (uint16_t)(man ? (sign | 0x7e00u | (man >> 13)) : (sign | 0x7c00u));
    int e = (int)exp - 127 + 15;
    if (e >= 31)
        return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10)
            return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t h = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (h & 1)))
            h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1)))
        h++;
    return (uint16_t)h;
}

float orc_f16_value(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    if (exp == 0x1f)
        return u2f(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        float v = (float)man * 5.9604644775390625e-08f; /* 2^-24, exact */
        return (sign ? -v : v);
    }
    return u2f(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

uint16_t orc_bf16_bits(float f)
{
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t round_bit = 0x8000u;
    if ((x & round_bit) && (x & (3 * round_bit - 1)))
        return (uint16_t)((x >> 16) + 1);
    return (uint16_t)(x >> 16);
}

float orc_bf16_value(uint16_t b) { return u2f((uint32_t)b << 16); }

/* FP8 codecs, src/float8.rs:52-131 (E4M3: bias 7, no inf, NaN = S.1111.111;
 * E5M2: bias 15, IEEE-style). Pinned by the fp8 conformance fixtures. */
float orc_fp8_value(int fmt, uint8_t bits)
{
    int e4 = (fmt == ORC_FP8E4M3);
    int man_bits = e4 ? 3 : 2, bias = e4 ? 7 : 15, maxe = e4 ? 15 : 31;
    int exp = (bits >> man_bits) & maxe;
    int man = bits & ((1 << man_bits) - 1);
    double sign = (bits & 0x80) ? -1.0 : 1.0;
    if (e4 ? (exp == maxe && man == 7) : (exp == maxe && man != 0))
        return NAN;
    if (!e4 && exp == maxe)
        return (float)(sign * INFINITY);
    double scale = (double)(1 << man_bits);
    double mag = exp == 0 ? (man / scale) * ldexp(1.0, 1 - bias) : (1.0 + man / scale) * ldexp(1.0, exp - bias);
    return (float)(sign * mag);
}

uint8_t orc_fp8_bits(int fmt, float x)
{
    int e4 = (fmt == ORC_FP8E4M3);
    int man_bits = e4 ? 3 : 2, bias = e4 ? 7 : 15, maxe = e4 ? 15 : 31;
    uint32_t man_mask = (1u << man_bits) - 1;
    uint8_t nan = (uint8_t)((maxe << man_bits) | man_mask);
    if (isnan(x))
        return nan;
    uint8_t sign = signbit(x) ? 0x80 : 0;
    uint8_t overflow = e4 ? (uint8_t)(sign | nan) : (uint8_t)(sign | (maxe << man_bits));
    if (isinf(x))
        return overflow;
    double a = fabs((double)x);
    if (a == 0.0)
        return sign;
    double man_scale = (double)(1 << man_bits);
    int min_normal_exp = 1 - bias;
    int e;
    frexp(a, &e);
    e -= 1; /* a = m * 2^e with m in [1,2) */
    uint32_t exp_field, man;
    if (e < min_normal_exp) {
        uint32_t q = (uint32_t)nearbyint(a / ldexp(1.0, min_normal_exp) * man_scale);
        exp_field = q >> man_bits;
        man = q & man_mask;
    } else {
        uint32_t q = (uint32_t)nearbyint(a / ldexp(1.0, e) * man_scale);
        if (q == (2u << man_bits)) {
            e += 1;
            q = 1u << man_bits;
        }
        exp_field = (uint32_t)(e + bias);
        man = q & man_mask;
    }
    int exceeded = e4 ? (exp_field > (uint32_t)maxe || (exp_field == (uint32_t)maxe && man == man_mask))
                      : (exp_field >= (uint32_t)maxe);
    if (exceeded)
        return overflow;
    return (uint8_t)(sign | (exp_field << man_bits) | man);
}

/* round_to, src/ops/common.rs:100-108 */
float orc_round_to(int fmt, float x)
{
    switch (fmt) {
    case ORC_F16: return orc_f16_value(orc_f16_bits(x));
    case ORC_BF16: return orc_bf16_value(orc_bf16_bits(x));
    case ORC_FP8E4M3:
    case ORC_FP8E5M2: return orc_fp8_value(fmt, orc_fp8_bits(fmt, x));
    default: return x;
    }
}

/* ---------------------------------------------------------------------------
 * Fixed-point scaling, src/ops/quant.rs.
 * ------------------------------------------------------------------------- */

/* reciprocal_scale, src/ops/quant.rs:6-11. Pinned by the reference's own
 * known-answer test (quant.rs:38-48) restated in tests/test_oracle.py and by
 * the int8/int16 AVG_POOL2D fixtures. */
int32_t orc_reciprocal_scale(int32_t value, int32_t *shift)
{
    uint32_t v1 = (uint32_t)value - 1u;
    int lz = v1 == 0 ? 32 : __builtin_clz(v1);
    int k = 32 - lz;
    int64_t numerator = ((int64_t)(1LL << 30) + 1) << k;
    *shift = 30 + k;
    return (int32_t)(numerator / (int64_t)value);
}

/* apply_scale_32, src/ops/quant.rs:17-32: REQUIRE failures return ORC_ERR. */
int orc_apply_scale_32(int32_t value, int32_t multiplier, int32_t shift, int double_round, int32_t *out)
{
    if (multiplier < 0 || shift < 2 || shift > 62)
        return ORC_ERR;
    int64_t low = -(int64_t)(1ULL << (shift - 1)), high = (int64_t)(1ULL << (shift - 1));
    int64_t v = value;
    if (v < low || v >= high)
        return ORC_ERR;
    int64_t round = (int64_t)(1ULL << (shift - 1));
    if (double_round && shift > 31)
        round += v >= 0 ? (1LL << 30) : -(1LL << 30);
    int64_t result = (v * (int64_t)multiplier + round) >> shift;
    if (result < INT32_MIN || result > INT32_MAX)
        return ORC_ERR;
    *out = (int32_t)result;
    return ORC_OK;
}

/* apply_scale_16, src/ops/type_conv.rs:86-92 */
int orc_apply_scale_16(int64_t value, int16_t multiplier, int32_t shift, int32_t *out)
{
    if (multiplier < 0 || shift < 2 || shift > 62)
        return ORC_ERR;
    int64_t result = (int64_t)((uint64_t)value * (uint64_t)(int64_t)multiplier + (1ULL << (shift - 1))) >> shift;
    if (result < INT32_MIN || result > INT32_MAX)
        return ORC_ERR;
    *out = (int32_t)result;
    return ORC_OK;
}

/* ---------------------------------------------------------------------------
 * Accumulators, src/ops/accum.rs:20-139.
 * ------------------------------------------------------------------------- */
enum { ACC_I32 = 0, ACC_I48 = 1 };
enum { FACC_F32 = 0, FACC_F16 = 1, FACC_BF16 = 2, FACC_F16U = 3, FACC_BF16U = 4 };

static inline float facc_mac(int kind, float acc, float a, float b)
{
    switch (kind) {
    case FACC_F16: return orc_round_to(ORC_F16, acc + orc_round_to(ORC_F16, a * b)); /* accum.rs:86-89 */
    case FACC_BF16: return orc_round_to(ORC_BF16, acc + orc_round_to(ORC_BF16, a * b)); /* accum.rs:135-138 */
    case FACC_F16U: return orc_round_to(ORC_F16, acc + a * b); /* accum.rs:103-106 */
    case FACC_BF16U: return orc_round_to(ORC_BF16, acc + a * b); /* accum.rs:119-122 */
    default: return acc + a * b; /* accum.rs:68-70 */
    }
}

static int64_t clamp48(int64_t v)
{
    const int64_t lo = -(1LL << 47), hi = (1LL << 47) - 1;
    return v < lo ? lo : (v > hi ? hi : v);
}

/* Geometry shared by CONV2D / DEPTHWISE_CONV2D: out = (in-1+pb+pa-(k-1)*d)/s+1
 * (src/ops/conv.rs:57-75). The caller has validated it. */
static int conv_extent(int in, int pb, int pa, int k, int d, int s)
{
    return (in - 1 + pb + pa - (k - 1) * d) / s + 1;
}

/* CONV2D integer branch: src/ops/conv.rs:149-181 (loop order) and :457-474
 * (zero points, bias, INT48 clamp). Pinned by the i8xi8, i8xi4 and i16xi8
 * conv2d fixtures and a numpy brute force. */
void orc_conv2d_int(const int64_t *x, const int64_t *w, const int64_t *bias, int bias_len, int n, int ih, int iw,
                    int ic, int oc, int kh, int kw, const int32_t *pad, const int32_t *stride, const int32_t *dil,
                    int64_t in_zp, int64_t w_zp, int acc_kind, int64_t *out)
{
    int oh = conv_extent(ih, pad[0], pad[1], kh, dil[0], stride[0]);
    int ow = conv_extent(iw, pad[2], pad[3], kw, dil[1], stride[1]);
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++)
                for (int co = 0; co < oc; co++) {
                    uint32_t acc32 = 0;
                    uint64_t acc64 = 0;
                    for (int ky = 0; ky < kh; ky++) {
                        int y = oy * stride[0] + ky * dil[0] - pad[0];
                        if (y < 0 || y >= ih)
                            continue;
                        for (int kx = 0; kx < kw; kx++) {
                            int xx = ox * stride[1] + kx * dil[1] - pad[2];
                            if (xx < 0 || xx >= iw)
                                continue;
                            const int64_t *xi = x + (((int64_t)b * ih + y) * iw + xx) * ic;
                            const int64_t *wi = w + (((int64_t)co * kh + ky) * kw + kx) * ic;
                            for (int c = 0; c < ic; c++) {
                                if (acc_kind == ACC_I32) {
                                    uint32_t a = (uint32_t)(int32_t)(xi[c] - in_zp);
                                    uint32_t bb = (uint32_t)(int32_t)(wi[c] - w_zp);
                                    acc32 += a * bb;
                                } else {
                                    acc64 += (uint64_t)(xi[c] - in_zp) * (uint64_t)(wi[c] - w_zp);
                                }
                            }
                        }
                    }
                    int64_t bv = bias[bias_len == 1 ? 0 : co];
                    if (acc_kind == ACC_I32)
                        out[o++] = (int32_t)(acc32 + (uint32_t)(int32_t)bv);
                    else
                        out[o++] = clamp48((int64_t)(acc64 + (uint64_t)bv));
                }
}

/* CONV2D float branch: src/ops/conv.rs:475-496 with ConvNd::accumulate's
 * order (:149-181); acc kinds as accum.rs. out = round(round(acc)+bias). */
void orc_conv2d_float(const float *x, const float *w, const float *bias, int bias_len, int n, int ih, int iw, int ic,
                      int oc, int kh, int kw, const int32_t *pad, const int32_t *stride, const int32_t *dil, float in_zp,
                      float w_zp, int acc_kind, int out_fmt, float *out)
{
    int oh = conv_extent(ih, pad[0], pad[1], kh, dil[0], stride[0]);
    int ow = conv_extent(iw, pad[2], pad[3], kw, dil[1], stride[1]);
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++)
                for (int co = 0; co < oc; co++) {
                    float acc = 0.0f;
                    for (int ky = 0; ky < kh; ky++) {
                        int y = oy * stride[0] + ky * dil[0] - pad[0];
                        if (y < 0 || y >= ih)
                            continue;
                        for (int kx = 0; kx < kw; kx++) {
                            int xx = ox * stride[1] + kx * dil[1] - pad[2];
                            if (xx < 0 || xx >= iw)
                                continue;
                            const float *xi = x + (((int64_t)b * ih + y) * iw + xx) * ic;
                            const float *wi = w + (((int64_t)co * kh + ky) * kw + kx) * ic;
                            for (int c = 0; c < ic; c++)
                                acc = facc_mac(acc_kind, acc, xi[c] - in_zp, wi[c] - w_zp);
                        }
                    }
                    float bv = bias[bias_len == 1 ? 0 : co];
                    out[o++] = orc_round_to(out_fmt, orc_round_to(out_fmt, acc) + bv);
                }
}

/* DEPTHWISE_CONV2D: src/ops/conv.rs:234-266 (weight [KH,KW,C,M], output
 * channel c*M+m) with eval_conv's integer epilogue (:457-474). */
void orc_depthwise_int(const int64_t *x, const int64_t *w, const int64_t *bias, int bias_len, int n, int ih, int iw,
                       int c, int m, int kh, int kw, const int32_t *pad, const int32_t *stride, const int32_t *dil,
                       int64_t in_zp, int64_t w_zp, int acc_kind, int64_t *out)
{
    int oh = conv_extent(ih, pad[0], pad[1], kh, dil[0], stride[0]);
    int ow = conv_extent(iw, pad[2], pad[3], kw, dil[1], stride[1]);
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++)
                for (int ci = 0; ci < c; ci++)
                    for (int mi = 0; mi < m; mi++) {
                        uint32_t acc32 = 0;
                        uint64_t acc64 = 0;
                        for (int ky = 0; ky < kh; ky++) {
                            int y = oy * stride[0] - pad[0] + ky * dil[0];
                            if (y < 0 || y >= ih)
                                continue;
                            for (int kx = 0; kx < kw; kx++) {
                                int xx = ox * stride[1] - pad[2] + kx * dil[1];
                                if (xx < 0 || xx >= iw)
                                    continue;
                                int64_t xv = x[(((int64_t)b * ih + y) * iw + xx) * c + ci];
                                int64_t wv = w[(((int64_t)ky * kw + kx) * c + ci) * m + mi];
                                if (acc_kind == ACC_I32)
                                    acc32 += (uint32_t)(int32_t)(xv - in_zp) * (uint32_t)(int32_t)(wv - w_zp);
                                else
                                    acc64 += (uint64_t)(xv - in_zp) * (uint64_t)(wv - w_zp);
                            }
                        }
                        int64_t bv = bias[bias_len == 1 ? 0 : ci * m + mi];
                        if (acc_kind == ACC_I32)
                            out[o++] = (int32_t)(acc32 + (uint32_t)(int32_t)bv);
                        else
                            out[o++] = clamp48((int64_t)(acc64 + (uint64_t)bv));
                    }
}

void orc_depthwise_float(const float *x, const float *w, const float *bias, int bias_len, int n, int ih, int iw, int c,
                         int m, int kh, int kw, const int32_t *pad, const int32_t *stride, const int32_t *dil,
                         float in_zp, float w_zp, int acc_kind, int out_fmt, float *out)
{
    int oh = conv_extent(ih, pad[0], pad[1], kh, dil[0], stride[0]);
    int ow = conv_extent(iw, pad[2], pad[3], kw, dil[1], stride[1]);
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++)
                for (int ci = 0; ci < c; ci++)
                    for (int mi = 0; mi < m; mi++) {
                        float acc = 0.0f;
                        for (int ky = 0; ky < kh; ky++) {
                            int y = oy * stride[0] - pad[0] + ky * dil[0];
                            if (y < 0 || y >= ih)
                                continue;
                            for (int kx = 0; kx < kw; kx++) {
                                int xx = ox * stride[1] - pad[2] + kx * dil[1];
                                if (xx < 0 || xx >= iw)
                                    continue;
                                float xv = x[(((int64_t)b * ih + y) * iw + xx) * c + ci];
                                float wv = w[(((int64_t)ky * kw + kx) * c + ci) * m + mi];
                                acc = facc_mac(acc_kind, acc, xv - in_zp, wv - w_zp);
                            }
                        }
                        float bv = bias[bias_len == 1 ? 0 : ci * m + mi];
                        out[o++] = orc_round_to(out_fmt, orc_round_to(out_fmt, acc) + bv);
                    }
}

/* MATMUL integer: src/ops/matmul.rs:80-95 and :139-153. */
void orc_matmul_int(const int64_t *a, const int64_t *b, int n, int h, int c, int w, int64_t a_zp, int64_t b_zp,
                    int acc_kind, int64_t *out)
{
    int64_t o = 0;
    for (int bn = 0; bn < n; bn++)
        for (int row = 0; row < h; row++)
            for (int col = 0; col < w; col++) {
                uint32_t acc32 = 0;
                uint64_t acc64 = 0;
                for (int k = 0; k < c; k++) {
                    int64_t av = a[((int64_t)bn * h + row) * c + k] - a_zp;
                    int64_t bv = b[((int64_t)bn * c + k) * w + col] - b_zp;
                    if (acc_kind == ACC_I32)
                        acc32 += (uint32_t)(int32_t)av * (uint32_t)(int32_t)bv;
                    else
                        acc64 += (uint64_t)av * (uint64_t)bv;
                }
                out[o++] = acc_kind == ACC_I32 ? (int64_t)(int32_t)acc32 : clamp48((int64_t)acc64);
            }
}

/* MATMUL float: src/ops/matmul.rs:154-170; operands are pre-rounded to the
 * output type by the caller (`convert`, :160-162). */
void orc_matmul_float(const float *a, const float *b, int n, int h, int c, int w, int acc_kind, float *out)
{
    int64_t o = 0;
    for (int bn = 0; bn < n; bn++)
        for (int row = 0; row < h; row++)
            for (int col = 0; col < w; col++) {
                float acc = 0.0f;
                for (int k = 0; k < c; k++)
                    acc = facc_mac(acc_kind, acc, a[((int64_t)bn * h + row) * c + k], b[((int64_t)bn * c + k) * w + col]);
                out[o++] = acc;
            }
}

/* CONV3D: ConvNd::accumulate with three spatial dimensions
 * (src/ops/conv.rs:149-181: batch, output position (d, y, x), oc, then the
 * kernel position row-major (kd, ky, kx) and ic innermost), eval_conv's
 * epilogue (:457-496). x [N,ID,IH,IW,IC], w [OC,KD,KH,KW,IC]; pad
 * {front, back, top, bottom, left, right}, stride/dil {d, y, x}. `is_int`
 * selects the integer branch (xi/wi/bi, acc_kind ACC_I32/ACC_I48) or the
 * float one (xf/wf/bf, acc_kind FACC_*, out_fmt). */
void orc_conv3d(int is_int, const int64_t *xi, const int64_t *wi, const int64_t *bi, const float *xf, const float *wf,
                const float *bf, int bias_len, int n, int id, int ih, int iw, int ic, int oc, int kd, int kh, int kw,
                const int32_t *pad, const int32_t *stride, const int32_t *dil, int64_t in_zp, int64_t w_zp,
                int acc_kind, int out_fmt, int64_t *out_i, float *out_f)
{
    int od = conv_extent(id, pad[0], pad[1], kd, dil[0], stride[0]);
    int oh = conv_extent(ih, pad[2], pad[3], kh, dil[1], stride[1]);
    int ow = conv_extent(iw, pad[4], pad[5], kw, dil[2], stride[2]);
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oz = 0; oz < od; oz++)
            for (int oy = 0; oy < oh; oy++)
                for (int ox = 0; ox < ow; ox++)
                    for (int co = 0; co < oc; co++) {
                        uint32_t acc32 = 0;
                        uint64_t acc64 = 0;
                        float accf = 0.0f;
                        for (int kz = 0; kz < kd; kz++) {
                            int z = oz * stride[0] + kz * dil[0] - pad[0];
                            if (z < 0 || z >= id)
                                continue;
                            for (int ky = 0; ky < kh; ky++) {
                                int y = oy * stride[1] + ky * dil[1] - pad[2];
                                if (y < 0 || y >= ih)
                                    continue;
                                for (int kx = 0; kx < kw; kx++) {
                                    int xx = ox * stride[2] + kx * dil[2] - pad[4];
                                    if (xx < 0 || xx >= iw)
                                        continue;
                                    int64_t xb = ((((int64_t)b * id + z) * ih + y) * iw + xx) * ic;
                                    int64_t wb = ((((int64_t)co * kd + kz) * kh + ky) * kw + kx) * ic;
                                    for (int c = 0; c < ic; c++) {
                                        if (!is_int) {
                                            accf = facc_mac(acc_kind, accf, xf[xb + c], wf[wb + c]);
                                        } else if (acc_kind == ACC_I32) {
                                            acc32 += (uint32_t)(int32_t)(xi[xb + c] - in_zp) *
                                                     (uint32_t)(int32_t)(wi[wb + c] - w_zp);
                                        } else {
                                            acc64 += (uint64_t)(xi[xb + c] - in_zp) * (uint64_t)(wi[wb + c] - w_zp);
                                        }
                                    }
                                }
                            }
                        }
                        int bidx = bias_len == 1 ? 0 : co;
                        if (!is_int)
                            out_f[o++] = orc_round_to(out_fmt, orc_round_to(out_fmt, accf) + bf[bidx]);
                        else if (acc_kind == ACC_I32)
                            out_i[o++] = (int32_t)(acc32 + (uint32_t)(int32_t)bi[bidx]);
                        else
                            out_i[o++] = clamp48((int64_t)(acc64 + (uint64_t)bi[bidx]));
                    }
}

/* TRANSPOSE_CONV2D: Transpose::accumulate, the gather form
 * (src/ops/conv.rs:337-372: output (oy, ox) reads input
 * ((oy - out_pad_top - ky) / sy, (ox - out_pad_left - kx) / sx) where the
 * division is exact and in range; oc, then ky, kx, ic innermost) with
 * eval_conv's epilogue (:457-496). x [N,IH,IW,IC], w [OC,KH,KW,IC];
 * out_pad {top, bottom, left, right} (may be negative); output extent
 * (I-1)*s + pad_a + pad_b + K (:302-304). Branches as orc_conv3d. */
void orc_transpose_conv2d(int is_int, const int64_t *xi, const int64_t *wi, const int64_t *bi, const float *xf,
                          const float *wf, const float *bf, int bias_len, int n, int ih, int iw, int ic, int oc,
                          int kh, int kw, const int32_t *out_pad, const int32_t *stride, int64_t in_zp, int64_t w_zp,
                          int acc_kind, int out_fmt, int64_t *out_i, float *out_f)
{
    int oh = (ih - 1) * stride[0] + out_pad[0] + out_pad[1] + kh;
    int ow = (iw - 1) * stride[1] + out_pad[2] + out_pad[3] + kw;
    int sy = stride[0], sx = stride[1];
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oy = 0; oy < oh; oy++) {
            int iy = oy - out_pad[0];
            for (int ox = 0; ox < ow; ox++) {
                int ix = ox - out_pad[2];
                for (int co = 0; co < oc; co++) {
                    uint32_t acc32 = 0;
                    uint64_t acc64 = 0;
                    float accf = 0.0f;
                    for (int ky = 0; ky < kh; ky++) {
                        int y = iy - ky;
                        if (y < 0 || y >= ih * sy || y % sy != 0)
                            continue;
                        for (int kx = 0; kx < kw; kx++) {
                            int xx = ix - kx;
                            if (xx < 0 || xx >= iw * sx || xx % sx != 0)
                                continue;
                            int64_t xb = (((int64_t)b * ih + y / sy) * iw + xx / sx) * ic;
                            int64_t wb = (((int64_t)co * kh + ky) * kw + kx) * ic;
                            for (int c = 0; c < ic; c++) {
                                if (!is_int) {
                                    accf = facc_mac(acc_kind, accf, xf[xb + c], wf[wb + c]);
                                } else if (acc_kind == ACC_I32) {
                                    acc32 += (uint32_t)(int32_t)(xi[xb + c] - in_zp) *
                                             (uint32_t)(int32_t)(wi[wb + c] - w_zp);
                                } else {
                                    acc64 += (uint64_t)(xi[xb + c] - in_zp) * (uint64_t)(wi[wb + c] - w_zp);
                                }
                            }
                        }
                    }
                    int bidx = bias_len == 1 ? 0 : co;
                    if (!is_int)
                        out_f[o++] = orc_round_to(out_fmt, orc_round_to(out_fmt, accf) + bf[bidx]);
                    else if (acc_kind == ACC_I32)
                        out_i[o++] = (int32_t)(acc32 + (uint32_t)(int32_t)bi[bidx]);
                    else
                        out_i[o++] = clamp48((int64_t)(acc64 + (uint64_t)bi[bidx]));
                }
            }
        }
}

/* AVG_POOL2D integer: src/ops/pool.rs:193-214 with for_each_window (:77-104).
 * Returns ORC_ERR where apply_scale_32 would (a REQUIRE failure). */
int orc_avg_pool_int(const int64_t *x, int n, int ih, int iw, int c, const int32_t *kernel, const int32_t *stride,
                     const int32_t *pad, int64_t in_zp, int64_t out_zp, int64_t lo, int64_t hi, int64_t *out)
{
    int oh = (ih + pad[0] + pad[1] - kernel[0]) / stride[0] + 1;
    int ow = (iw + pad[2] + pad[3] - kernel[1]) / stride[1] + 1;
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++)
                for (int ci = 0; ci < c; ci++) {
                    uint32_t acc = 0;
                    int32_t count = 0;
                    for (int ky = 0; ky < kernel[0]; ky++) {
                        int y = oy * stride[0] - pad[0] + ky;
                        if (y < 0 || y >= ih)
                            continue;
                        for (int kx = 0; kx < kernel[1]; kx++) {
                            int xx = ox * stride[1] - pad[2] + kx;
                            if (xx < 0 || xx >= iw)
                                continue;
                            acc += (uint32_t)(int32_t)(x[(((int64_t)b * ih + y) * iw + xx) * c + ci] - in_zp);
                            count++;
                        }
                    }
                    int32_t shift, v;
                    int32_t mult = orc_reciprocal_scale(count, &shift);
                    if (orc_apply_scale_32((int32_t)acc, mult, shift, 0, &v) != ORC_OK)
                        return ORC_ERR;
                    int64_t r = (int64_t)v + out_zp;
                    out[o++] = r < lo ? lo : (r > hi ? hi : r);
                }
    return ORC_OK;
}

/* AVG_POOL2D float: src/ops/pool.rs:215-227: every add and the divide are
 * rounded to acc_t; the caller encodes the result in the input type. */
void orc_avg_pool_float(const float *x, int n, int ih, int iw, int c, const int32_t *kernel, const int32_t *stride,
                        const int32_t *pad, int acc_fmt, float *out)
{
    int oh = (ih + pad[0] + pad[1] - kernel[0]) / stride[0] + 1;
    int ow = (iw + pad[2] + pad[3] - kernel[1]) / stride[1] + 1;
    int64_t o = 0;
    for (int b = 0; b < n; b++)
        for (int oy = 0; oy < oh; oy++)
            for (int ox = 0; ox < ow; ox++)
                for (int ci = 0; ci < c; ci++) {
                    float acc = 0.0f;
                    int count = 0;
                    for (int ky = 0; ky < kernel[0]; ky++) {
                        int y = oy * stride[0] - pad[0] + ky;
                        if (y < 0 || y >= ih)
                            continue;
                        for (int kx = 0; kx < kernel[1]; kx++) {
                            int xx = ox * stride[1] - pad[2] + kx;
                            if (xx < 0 || xx >= iw)
                                continue;
                            acc = orc_round_to(acc_fmt, acc + x[(((int64_t)b * ih + y) * iw + xx) * c + ci]);
                            count++;
                        }
                    }
                    out[o++] = orc_round_to(acc_fmt, acc / (float)count);
                }
}

/* RESCALE per element: src/ops/type_conv.rs:171-188 (after the operand
 * checks of :117-170, which the caller has done). Rounding modes: 1 SINGLE,
 * 2 INEXACT, 3 DOUBLE (schema/tosa.fbs:59-64). in_bits/out_bits are the
 * type widths (8, 16, 32, 48). Returns ORC_ERR on a REQUIRE failure. */
static int64_t extend(int bits, int64_t v, int unsigned_)
{
    return unsigned_ ? (v & (int64_t)((1ULL << bits) - 1)) : v;
}

static int32_t sat_f32_to_i32(float f)
{
    if (isnan(f))
        return 0;
    if (f >= 2147483648.0f)
        return INT32_MAX;
    if (f < -2147483648.0f)
        return INT32_MIN;
    return (int32_t)f;
}

int orc_rescale(const int64_t *x, int64_t count, const int64_t *mult, const int64_t *shift, int64_t channels,
                int per_channel, int scale32, int rounding, int in_bits, int out_bits, int in_unsigned,
                int out_unsigned, int64_t in_zp_raw, int64_t out_zp_raw, int64_t *out)
{
    int64_t in_zp = extend(in_bits, in_zp_raw, in_unsigned);
    int64_t out_zp = extend(out_bits, out_zp_raw, out_unsigned);
    int64_t lo, hi;
    if (out_unsigned) {
        lo = 0;
        hi = (int64_t)((1ULL << out_bits) - 1);
    } else {
        lo = -(int64_t)(1ULL << (out_bits - 1));
        hi = (int64_t)(1ULL << (out_bits - 1)) - 1;
    }
    for (int64_t i = 0; i < count; i++) {
        int64_t ch = per_channel ? i % channels : 0;
        int32_t m = (int32_t)mult[ch], s = (int32_t)shift[ch];
        int64_t v = extend(in_bits, x[i], in_unsigned) - in_zp;
        int32_t scaled;
        if (rounding == 2) {
            float p = (float)v * (float)m;
            scaled = sat_f32_to_i32(nearbyintf(p * ldexpf(1.0f, -s)));
        } else if (scale32) {
            if (orc_apply_scale_32((int32_t)v, m, s, rounding == 3, &scaled) != ORC_OK)
                return ORC_ERR;
        } else {
            if (orc_apply_scale_16(v, (int16_t)m, s, &scaled) != ORC_OK)
                return ORC_ERR;
        }
        int64_t r = (int64_t)scaled + out_zp;
        if (r < INT32_MIN || r > INT32_MAX)
            return ORC_ERR;
        out[i] = r < lo ? lo : (r > hi ? hi : r);
    }
    return ORC_OK;
}

/* Array forms of the codecs, for the Python side. */
void orc_encode_array(int fmt, const float *x, int64_t n, void *out)
{
    for (int64_t i = 0; i < n; i++) {
        if (fmt == ORC_F16)
            ((uint16_t *)out)[i] = orc_f16_bits(x[i]);
        else if (fmt == ORC_BF16)
            ((uint16_t *)out)[i] = orc_bf16_bits(x[i]);
        else if (fmt == ORC_FP8E4M3 || fmt == ORC_FP8E5M2)
            ((uint8_t *)out)[i] = orc_fp8_bits(fmt, x[i]);
        else
            ((float *)out)[i] = x[i];
    }
}

void orc_decode_array(int fmt, const void *in, int64_t n, float *out)
{
    for (int64_t i = 0; i < n; i++) {
        if (fmt == ORC_F16)
            out[i] = orc_f16_value(((const uint16_t *)in)[i]);
        else if (fmt == ORC_BF16)
            out[i] = orc_bf16_value(((const uint16_t *)in)[i]);
        else if (fmt == ORC_FP8E4M3 || fmt == ORC_FP8E5M2)
            out[i] = orc_fp8_value(fmt, ((const uint8_t *)in)[i]);
        else
            out[i] = ((const float *)in)[i];
    }
}

void orc_round_array(int fmt, const float *x, int64_t n, float *out)
{
    for (int64_t i = 0; i < n; i++)
        out[i] = orc_round_to(fmt, x[i]);
}
