// Op-level entry points of the C ABI: one int8 CONV2D, optionally followed
// by the RESCALE (and CLAMP) that come after it in a quantised graph, on
// caller-owned device buffers and without a graph.
//
// They stand for the reference's per-operator boundary, ops::dispatch
// (src/ops/mod.rs:22), reaching eval_conv's integer branch
// (src/ops/conv.rs:398-474), eval_rescale (src/ops/type_conv.rs:111-191) and
// eval_clamp (src/ops/elementwise.rs:314-343). The checks are the graph
// path's: ConvNd::new's ERROR_IF (src/ops/conv.rs:57-139) and RESCALE's
// parameter checks; the kernels are the graph path's fused ones (epilogue
// table, packed weights, conv_i8_fast).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/tosa_mi355x.h"
#include "core.h"
#include "device.h"
#include "kernels.h"
#include "opapi.h"

namespace tosa {
namespace {

using kern::ConvI8Desc;
using kern::RescaleDev;

constexpr const char* OP = "CONV2D";

Error bad_arg(const std::string& m) { return Error(static_cast<ErrorKind>(TOSA_ERR_INVALID_ARGUMENT), m); }

int64_t extent(int64_t in, int32_t pb, int32_t pa, int64_t k, int32_t d, int32_t s)
{
    const int64_t full = in - 1 + pb + pa - (k - 1) * d;
    if (full % s != 0)
        throw invalid(OP, "parameters must yield exact integer output dimensions");
    const int64_t out = full / s + 1;
    if (out < 1)
        throw invalid(OP, "output dimension " + std::to_string(out) + " must be positive");
    return out;
}

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Workspace of tosa_conv2d_i8_noalloc: one array per GPU, for the life of
// the process. Its first 256 bytes are a discard error word (written by no
// kernel in the calls that use it: those without a RESCALE); the rest holds
// one call's workspace. Host code never passes the array's name to a kernel
// (on the host it is a stand-in, not a device address): it uses the address
// hipGetSymbolAddress reports for the current device.
constexpr size_t SCRATCH_BYTES = size_t(4) << 20;
constexpr size_t SCRATCH_WORKSPACE = SCRATCH_BYTES - 256;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[MAX_DEVICES] = {};

// The device address of `scratch` on the current device, looked up once per
// device (each GPU holds its own copy at its own address).
uint8_t* scratch_on_current_device()
{
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= MAX_DEVICES)
        throw Error(ERR_DEVICE, "device index " + std::to_string(dev) + " beyond the scratch table");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            throw Error(ERR_DEVICE, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
    }
    return g_scratch_ptr[dev];
}

// RESCALE multiplier/shift words written into device memory from the
// kernel's own arguments (no staging buffer, nothing a graph capture could
// not record).
constexpr int PARAM_WORDS = 240;
struct ParamWords {
    int32_t v[PARAM_WORDS];
    int32_t n;
};

__global__ void __launch_bounds__(256) put_param_words(int32_t* dst, ParamWords p)
{
    const int i = int(threadIdx.x);
    if (i < p.n)
        dst[i] = p.v[i];
}

void upload_words(const std::vector<int32_t>& words, int32_t* dst, hipStream_t s)
{
    for (size_t i0 = 0; i0 < words.size(); i0 += PARAM_WORDS) {
        ParamWords p{};
        p.n = int32_t(std::min<size_t>(PARAM_WORDS, words.size() - i0));
        std::memcpy(p.v, words.data() + i0, size_t(p.n) * sizeof(int32_t));
        hipLaunchKernelGGL(put_param_words, dim3(1), dim3(256), 0, s, dst + i0, p);
    }
}

// RESCALE (and CLAMP) parameters of an op-level call: eval_rescale's checks
// for an int32 input with scale32 and input zero point 0
// (src/ops/type_conv.rs:111-191), apply_scale_32's parameter REQUIRE
// (src/ops/quant.rs:17-32) when there is any output, CLAMP's bounds
// (src/ops/elementwise.rs:314-343). `params` receives the multipliers, then
// the shifts, as int32 words.
void parse_rescale(const tosa_rescale_i32& r, int64_t oc, int64_t count, RescaleDev& rs, std::vector<int32_t>& params)
{
    const std::string RS = "RESCALE";
    if (!r.multiplier || !r.shift)
        throw bad_arg(RS + ": null multiplier or shift");
    if (r.channels != 1 && r.channels != oc)
        throw invalid(RS, "multiplier and shift must have 1 or " + std::to_string(oc) + " elements");
    const DType out_t = static_cast<DType>(r.output_dtype);
    if (out_t != DT_INT8 && out_t != DT_INT16 && out_t != DT_INT32)
        throw Error(ERR_DTYPE_MISMATCH, RS + ": unsupported types INT32 -> " + dtype_name(out_t));
    if (out_t == DT_INT8 ? (r.output_zp < -128 || r.output_zp > 127) : r.output_zp != 0)
        throw invalid(RS, "zero point not allowed for this type");
    rs.channels = r.channels;
    rs.per_channel = r.channels > 1 ? 1 : 0;
    rs.scale32 = 1;
    rs.rounding = r.double_round ? 3 : 1;
    rs.in_bits = 32;
    rs.in_unsigned = 0;
    rs.in_zp = 0;
    rs.out_zp = r.output_zp;
    const int bits = out_t == DT_INT8 ? 8 : out_t == DT_INT16 ? 16 : 32;
    rs.lo = -(int64_t(1) << (bits - 1));
    rs.hi = (int64_t(1) << (bits - 1)) - 1;
    rs.out_bytes = bits / 8;
    if (r.has_clamp) {
        if (r.clamp_min < rs.lo || r.clamp_max > rs.hi)
            throw invalid("CLAMP", "min_val and max_val must be values of the output type");
        if (r.clamp_max < r.clamp_min)
            throw invalid("CLAMP", "max_val must not be smaller than min_val");
        rs.has_clamp = 1;
        rs.clamp_lo = r.clamp_min;
        rs.clamp_hi = r.clamp_max;
    }
    rs.max_shift = 2;
    rs.min_shift = 62;
    params.resize(size_t(2 * r.channels));
    for (int32_t i = 0; i < r.channels; i++) {
        const int32_t m = r.multiplier[i], sh = r.shift[i];
        if (count > 0 && (m < 0 || sh < 2 || sh > 62))
            throw Error(ERR_GRAPH, "apply_scale_32: invalid multiplier " + std::to_string(m) + " or shift " +
                                       std::to_string(sh));
        params[size_t(i)] = m;
        params[size_t(r.channels + i)] = sh;
        rs.max_shift = std::max(rs.max_shift, sh);
        rs.min_shift = std::min(rs.min_shift, sh);
    }
}

}  // namespace

ConvI8Call prepare_conv2d_i8(const ConvI8Args& a)
{
    ConvI8Call c;
    if (!a.x || !a.w || !a.bias || !a.x_shape || !a.w_shape || !a.pad || !a.stride || !a.dilation)
        throw bad_arg(std::string(OP) + ": null operand or attribute pointer");
    for (int i = 0; i < 4; i++)
        if (a.x_shape[i] < 1 || a.w_shape[i] < 1)
            throw Error(ERR_SHAPE_MISMATCH, std::string(OP) + ": every input and weight dimension must be positive");
    if (a.w_shape[3] != a.x_shape[3])
        throw Error(ERR_SHAPE_MISMATCH, std::string(OP) + ": weight input channels " + std::to_string(a.w_shape[3]) +
                                            " != input channels " + std::to_string(a.x_shape[3]));
    const int64_t oc = a.w_shape[0];
    if (a.bias_len != oc && a.bias_len != 1)
        throw Error(ERR_SHAPE_MISMATCH, std::string(OP) + ": bias channels " + std::to_string(a.bias_len) +
                                            " must be 1 or match output channels " + std::to_string(oc));
    for (int i = 0; i < 4; i++)
        if (a.pad[i] < 0)
            throw invalid(OP, "pad must be non-negative");
    for (int i = 0; i < 2; i++) {
        if (a.stride[i] < 1)
            throw invalid(OP, "stride must be at least 1");
        if (a.dilation[i] < 1)
            throw invalid(OP, "dilation must be at least 1");
    }
    if (a.input_zp < -128 || a.input_zp > 127 || a.weight_zp < -128 || a.weight_zp > 127)
        throw Error(ERR_DTYPE_MISMATCH, std::string(OP) + ": zero points must be int8 values");
    const int64_t oh = extent(a.x_shape[1], a.pad[0], a.pad[1], a.w_shape[1], a.dilation[0], a.stride[0]);
    const int64_t ow = extent(a.x_shape[2], a.pad[2], a.pad[3], a.w_shape[2], a.dilation[1], a.stride[1]);
    const int64_t n = a.x_shape[0], ih = a.x_shape[1], iw = a.x_shape[2], ic = a.x_shape[3];
    c.out_shape[0] = n;
    c.out_shape[1] = oh;
    c.out_shape[2] = ow;
    c.out_shape[3] = oc;
    c.count = n * oh * ow * oc;
    const int64_t K = a.w_shape[1] * a.w_shape[2] * ic;
    if (n * ih * iw * ic >= (int64_t(1) << 31) || c.count >= (int64_t(1) << 31) || K >= (int64_t(1) << 30) ||
        oc * K >= (int64_t(1) << 31))
        throw bad_arg(std::string(OP) + ": operands of 2^31 elements or more are not supported");

    ConvI8Desc& d = c.d;
    d.x = a.x;
    d.w = a.w;
    d.bias = a.bias;
    d.bias_len = int32_t(a.bias_len);
    d.n = int32_t(n);
    d.ih = int32_t(ih);
    d.iw = int32_t(iw);
    d.ic = int32_t(ic);
    d.oc = int32_t(oc);
    d.kh = int32_t(a.w_shape[1]);
    d.kw = int32_t(a.w_shape[2]);
    d.oh = int32_t(oh);
    d.ow = int32_t(ow);
    d.pt = a.pad[0];
    d.pl = a.pad[2];
    d.sy = a.stride[0];
    d.sx = a.stride[1];
    d.dy = a.dilation[0];
    d.dx = a.dilation[1];
    d.zp_x = a.input_zp;
    d.zp_w = a.weight_zp;
    if (!kern::conv_i8_fast_supported(d))
        throw Error(ERR_UNSUPPORTED_OP,
                    std::string(OP) + ": the op-level entry takes 16-byte aligned x and w, with input channels a "
                                      "multiple of 16 (1x1 stride 1 unpadded) or of 64 (any other geometry); "
                                      "other convolutions run through a graph");

    if (a.rescale) {
        parse_rescale(*a.rescale, oc, c.count, c.rs, c.params);
        c.has_rs = true;
        c.epi_ok = kern::conv_i8_fast_epilogue_ok(c.rs);
    }

    // Workspace layout: multiplier and shift words, the epilogue table,
    // the packed weights, and (a RESCALE the fused epilogue cannot take) the
    // int32 result.
    int64_t off = 0;
    c.params_off = off;
    off += round_up(int64_t(c.params.size()) * 4, 256);
    c.tab_off = off;
    off += round_up(kern::conv_i8_table_words(d.oc, 1) * 4, 256);
    c.wpack_bytes = kern::conv_i8_wpack_bytes(d);
    c.wpack_off = off;
    off += round_up(std::max<int64_t>(c.wpack_bytes, 0), 256);
    c.tmp_off = off;
    if (c.has_rs && !c.epi_ok)
        off += round_up(c.count * 4, 256);
    c.workspace = off;
    return c;
}

void launch_conv2d_i8(const ConvI8Call& c, uint8_t* ws, void* out, uint32_t* err, hipStream_t s)
{
    if (c.count == 0)
        return;
    ConvI8Desc d = c.d;
    RescaleDev rs = c.rs;
    if (c.has_rs) {
        rs.mult = reinterpret_cast<const int32_t*>(ws + c.params_off);
        rs.shift = rs.mult + rs.channels;
    }
    // The fused epilogue's table, or the plain int32 one when the RESCALE
    // runs as its own kernel afterwards.
    const RescaleDev* trs = c.has_rs && c.epi_ok ? &rs : nullptr;
    void* tab = ws + c.tab_off;
    kern::conv_i8_table(d, trs, tab, s);
    if (c.wpack_bytes > 0) {
        kern::conv_i8_wpack(d, ws + c.wpack_off, s);
        d.wpack = reinterpret_cast<const int8_t*>(ws + c.wpack_off);
    }
    if (!c.has_rs || c.epi_ok) {
        kern::conv_i8_fast(d, tab, trs, out, err, s);
        return;
    }
    void* tmp = ws + c.tmp_off;
    kern::conv_i8_fast(d, tab, nullptr, tmp, err, s);
    kern::rescale(rs, kern::E_I32, tmp, c.count, out, err, s);
}

void conv2d_i8(const ConvI8Args& a, int64_t* out_shape)
{
    const ConvI8Call c = prepare_conv2d_i8(a);
    if (out_shape)
        std::memcpy(out_shape, c.out_shape, sizeof c.out_shape);
    if (c.count == 0 || !a.out)
        return;  // nothing to compute, or a query of the output shape
    Stream& ts = thread_stream();
    const hipStream_t s = a.stream ? static_cast<hipStream_t>(a.stream) : ts.s;
    uint32_t* err = a.device_error;
    if (!err) {
        if (s != ts.s)
            throw bad_arg(std::string(OP) + ": device_error is required on a stream other than this thread's");
        err = ts.err;
    }
    // One pool block for the call, released stream-ordered after the
    // launches; the multiplier and shift words go up through pinned staging.
    auto* ws = static_cast<uint8_t*>(dev_alloc(size_t(c.workspace), s));
    if (!c.params.empty()) {
        const size_t bytes = c.params.size() * 4;
        void* h = pinned_acquire(bytes);
        std::memcpy(h, c.params.data(), bytes);
        hip_check(hipMemcpyAsync(ws + c.params_off, h, bytes, hipMemcpyHostToDevice, s), "upload RESCALE params");
        pinned_release(h, s);
    }
    launch_conv2d_i8(c, ws, a.out, err, s);
    dev_free(ws, size_t(c.workspace), s);
}

void conv2d_i8_noalloc(const ConvI8Args& a, int64_t* out_shape)
{
    const ConvI8Call c = prepare_conv2d_i8(a);
    if (out_shape)
        std::memcpy(out_shape, c.out_shape, sizeof c.out_shape);
    if (size_t(c.workspace) > SCRATCH_WORKSPACE)
        throw bad_arg(std::string(OP) + ": needs " + std::to_string(c.workspace) +
                      " bytes of workspace; tosa_conv2d_i8_noalloc holds at most " +
                      std::to_string(SCRATCH_WORKSPACE) + " (use tosa_conv2d_i8)");
    if (c.has_rs && !a.device_error)
        throw bad_arg(std::string(OP) + ": tosa_conv2d_i8_noalloc needs device_error with a RESCALE");
    if (c.count == 0 || !a.out)
        return;
    uint8_t* base = scratch_on_current_device();
    const hipStream_t s = static_cast<hipStream_t>(a.stream);  // NULL: HIP's null stream
    uint32_t* err = a.device_error ? a.device_error : reinterpret_cast<uint32_t*>(base);
    uint8_t* ws = base + 256;
    if (!c.params.empty())
        upload_words(c.params, reinterpret_cast<int32_t*>(ws + c.params_off), s);
    launch_conv2d_i8(c, ws, a.out, err, s);
}

void matmul_i8(const MatmulI8OpArgs& a, int64_t* out_shape)
{
    const std::string MM = "MATMUL";
    if (!a.a || !a.b || !a.a_shape || !a.b_shape)
        throw bad_arg(MM + ": null operand or shape pointer");
    for (int i = 0; i < 3; i++)
        if (a.a_shape[i] < 1 || a.b_shape[i] < 1)
            throw Error(ERR_SHAPE_MISMATCH, MM + ": every dimension of a and b must be positive");
    const int64_t n = a.a_shape[0], h = a.a_shape[1], c = a.a_shape[2], w = a.b_shape[2];
    // src/ops/matmul.rs:112-123: b is [N, C, W] with a's N and C.
    if (a.b_shape[0] != n || a.b_shape[1] != c)
        throw Error(ERR_SHAPE_MISMATCH, MM + ": b shape [" + std::to_string(a.b_shape[0]) + ", " +
                                            std::to_string(a.b_shape[1]) + ", " + std::to_string(w) +
                                            "] incompatible with a shape [" + std::to_string(n) + ", " +
                                            std::to_string(h) + ", " + std::to_string(c) + "]");
    if (a.a_zp < -128 || a.a_zp > 127 || a.b_zp < -128 || a.b_zp > 127)
        throw Error(ERR_DTYPE_MISMATCH, MM + ": zero points must be int8 values");
    const int64_t count = n * h * w;
    if (n * h * c >= (int64_t(1) << 31) || n * c * w >= (int64_t(1) << 31) || count >= (int64_t(1) << 31))
        throw bad_arg(MM + ": operands of 2^31 elements or more are not supported");
    if (out_shape) {
        out_shape[0] = n;
        out_shape[1] = h;
        out_shape[2] = w;
    }
    if (c > INT32_MAX || w > INT32_MAX ||
        !kern::matmul_i8_direct_applies(int32_t(c), int32_t(w), a.a, a.b))
        throw Error(ERR_UNSUPPORTED_OP, MM + ": the op-level entry takes 16-byte aligned a and b with C a multiple "
                                             "of 128 and W of 16; other shapes run through a graph");
    RescaleDev rs;
    std::vector<int32_t> params;
    if (a.rescale) {
        parse_rescale(*a.rescale, w, count, rs, params);
        if (!kern::conv_i8_fast_epilogue_ok(rs))
            throw Error(ERR_UNSUPPORTED_OP, MM + ": this RESCALE runs through a graph");
    }
    if (!a.out)
        return;  // a query of the output shape
    Stream& ts = thread_stream();
    const hipStream_t s = a.stream ? static_cast<hipStream_t>(a.stream) : ts.s;
    uint32_t* err = a.device_error;
    if (!err) {
        if (s != ts.s)
            throw bad_arg(MM + ": device_error is required on a stream other than this thread's");
        err = ts.err;
    }
    // Workspace: multiplier and shift words, then the epilogue table (the
    // bias-free additive constant C za zb and the RESCALE parameters; the
    // kernel adds the zero-point sums itself).
    const int64_t params_off = 0, tab_off = round_up(int64_t(params.size()) * 4, 256);
    const int64_t bytes = tab_off + round_up(kern::conv_i8_table_words(int32_t(w), 1) * 4, 256);
    auto* ws = static_cast<uint8_t*>(dev_alloc(size_t(bytes), s));
    if (!params.empty()) {
        const size_t pb = params.size() * 4;
        void* hp = pinned_acquire(pb);
        std::memcpy(hp, params.data(), pb);
        hip_check(hipMemcpyAsync(ws + params_off, hp, pb, hipMemcpyHostToDevice, s), "upload RESCALE params");
        pinned_release(hp, s);
        rs.mult = reinterpret_cast<const int32_t*>(ws + params_off);
        rs.shift = rs.mult + rs.channels;
    }
    ConvI8Desc td;
    td.x = a.a;
    td.w = nullptr;
    td.bias = nullptr;
    td.bias_len = 1;
    td.n = 1;
    td.ih = td.oh = int32_t(h);
    td.iw = td.ow = 1;
    td.ic = int32_t(c);
    td.oc = int32_t(w);
    td.zp_x = a.a_zp;
    td.zp_w = a.b_zp;
    td.batch = 1;
    kern::conv_i8_table(td, a.rescale ? &rs : nullptr, ws + tab_off, s);
    const bool done = kern::matmul_i8_direct(a.a, a.b, int32_t(n), int32_t(h), int32_t(c), int32_t(w), a.a_zp, a.b_zp,
                                             ws + tab_off, a.rescale ? &rs : nullptr, false, a.out, err, s);
    dev_free(ws, size_t(bytes), s);
    if (!done)
        throw Error(ERR_UNSUPPORTED_OP, MM + ": shape not taken by the one-kernel MATMUL");
}

}  // namespace tosa
