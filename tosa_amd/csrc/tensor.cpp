#include "tensor.h"

#include <cmath>
#include <cstring>

#include "device.h"

namespace tosa {

Storage::~Storage()
{
    if (ready)
        (void)hipEventDestroy(ready);
    if (dev && !external)
        dev_free(dev, dev_bytes, dev_stream);
}

static void ensure_alloc(Storage& s)
{
    if (s.dev)
        return;
    Stream& st = thread_stream();
    s.dev_bytes = s.bytes() ? s.bytes() : 1;
    s.dev_stream = st.s;
    s.dev = dev_alloc(s.dev_bytes, st.s);
}

// A stream other than the one that uploaded `s` waits for the upload.
static void order_after_upload(Storage& s)
{
    if (!s.ready)
        return;
    Stream& st = thread_stream();
    if (st.s != s.ready_stream)
        hip_check(hipStreamWaitEvent(st.s, s.ready, 0), "hipStreamWaitEvent(upload)");
}

const void* Storage::device_in()
{
    if (dev_valid.load(std::memory_order_acquire)) {
        if (ready) {
            std::lock_guard<std::recursive_mutex> lk(mu);
            order_after_upload(*this);
        }
        return dev;
    }
    std::lock_guard<std::recursive_mutex> lk(mu);
    if (dev_valid.load(std::memory_order_acquire)) {
        order_after_upload(*this);
        return dev;
    }
    if (host_valid) {
        ensure_alloc(*this);
        Stream& st = thread_stream();
        const size_t n = bytes();
        if (shared_const) {
            // A graph constant: any run, on any stream, may read it as soon as
            // dev_valid is set, so the copy completes first (once per graph).
            if (n)
                hip_check(hipMemcpyAsync(dev, host.data(), n, hipMemcpyHostToDevice, st.s), "upload constant");
            hip_check(hipStreamSynchronize(st.s), "hipStreamSynchronize(upload)");
        } else if (n) {
            // Through pinned staging: the copy is asynchronous for the host,
            // and the staging block is reused only once the stream has passed
            // the copy. Readers on other streams wait for `ready`.
            void* stage = pinned_acquire(n);
            std::memcpy(stage, host.data(), n);
            hip_check(hipMemcpyAsync(dev, stage, n, hipMemcpyHostToDevice, st.s), "upload tensor");
            pinned_release(stage, st.s);
            if (!ready)
                hip_check(hipEventCreateWithFlags(&ready, hipEventDisableTiming), "hipEventCreate(upload)");
            hip_check(hipEventRecord(ready, st.s), "hipEventRecord(upload)");
            ready_stream = st.s;
        }
        dev_valid.store(true, std::memory_order_release);
        return dev;
    }
    if (materialize) {
        auto f = materialize;  // keep the recipe alive while it runs
        f(*this);
        if (!dev_valid)
            throw Error(ERR_GRAPH, "internal error: a fused intermediate could not be recomputed");
        return dev;
    }
    throw Error(ERR_GRAPH, "internal error: tensor has no data");
}

void* Storage::device_out()
{
    std::lock_guard<std::recursive_mutex> lk(mu);
    ensure_alloc(*this);
    host_valid = false;
    dev_valid.store(true, std::memory_order_release);
    return dev;
}

const uint8_t* Storage::host_in()
{
    std::lock_guard<std::recursive_mutex> lk(mu);
    // Caller-owned device memory may have been rewritten since the last read:
    // its host mirror is never reused.
    if (host_valid && !external)
        return host.data();
    device_in();
    host.resize(bytes());
    Stream& st = thread_stream();
    if (bytes())
        hip_check(hipMemcpyAsync(host.data(), dev, bytes(), hipMemcpyDeviceToHost, st.s), "download tensor");
    hip_check(hipStreamSynchronize(st.s), "hipStreamSynchronize(download)");
    host_valid = true;
    return host.data();
}

StoragePtr make_host_storage(DType t, int64_t count, const void* data)
{
    auto s = std::make_shared<Storage>();
    s->dtype = t;
    s->count = count;
    s->host.resize(s->bytes());
    if (s->bytes() && data)
        std::memcpy(s->host.data(), data, s->bytes());
    s->host_valid = true;
    return s;
}

StoragePtr make_device_storage(DType t, int64_t count)
{
    auto s = std::make_shared<Storage>();
    s->dtype = t;
    s->count = count;
    ensure_alloc(*s);
    return s;
}

StoragePtr wrap_device_storage(DType t, int64_t count, void* dev_ptr)
{
    auto s = std::make_shared<Storage>();
    s->dtype = t;
    s->count = count;
    s->dev = dev_ptr;
    s->dev_bytes = s->bytes();
    s->external = true;
    s->dev_valid = true;
    return s;
}

std::vector<int64_t> int_values(const Tensor& t)
{
    const uint8_t* p = t.data->host_in();
    int64_t n = t.len();
    std::vector<int64_t> v(n);
    for (int64_t i = 0; i < n; i++) {
        switch (t.dtype()) {
        case DT_BOOL:
        case DT_INT4:
        case DT_INT8: v[i] = reinterpret_cast<const int8_t*>(p)[i]; break;
        case DT_INT16: v[i] = reinterpret_cast<const int16_t*>(p)[i]; break;
        case DT_INT32: v[i] = reinterpret_cast<const int32_t*>(p)[i]; break;
        case DT_INT48:
        case DT_INT64:
        case DT_SHAPE: v[i] = reinterpret_cast<const int64_t*>(p)[i]; break;
        default: throw Error(ERR_DTYPE_MISMATCH, std::string("not an integer tensor: ") + dtype_name(t.dtype()));
        }
    }
    if (t.dtype() == DT_BOOL)
        for (auto& x : v)
            x = x != 0;
    return v;
}

static float half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, man = h & 0x3ff, u;
    if (exp == 0x1f)
        u = sign | 0x7f800000u | (man << 13);
    else if (exp == 0) {
        float v = std::ldexp(static_cast<float>(man), -24);
        return sign ? -v : v;
    } else
        u = sign | ((exp + 112) << 23) | (man << 13);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

static double fp8_to_double(uint8_t b, bool e4m3)
{
    int mb = e4m3 ? 3 : 2, bias = e4m3 ? 7 : 15, maxe = e4m3 ? 15 : 31;
    int e = (b >> mb) & maxe, m = b & ((1 << mb) - 1);
    double sign = (b & 0x80) ? -1.0 : 1.0;
    if (e4m3 ? (e == 15 && m == 7) : (e == 31 && m != 0))
        return NAN;
    if (!e4m3 && e == 31)
        return sign * INFINITY;
    double mag = e == 0 ? std::ldexp(m, 1 - bias - mb) : std::ldexp((1 << mb) + m, e - bias - mb);
    return sign * mag;
}

std::vector<double> float_values(const Tensor& t)
{
    const uint8_t* p = t.data->host_in();
    int64_t n = t.len();
    std::vector<double> v(n);
    for (int64_t i = 0; i < n; i++) {
        switch (t.dtype()) {
        case DT_FP32: v[i] = reinterpret_cast<const float*>(p)[i]; break;
        case DT_FP16: v[i] = half_to_float(reinterpret_cast<const uint16_t*>(p)[i]); break;
        case DT_BF16: {
            uint32_t u = static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(p)[i]) << 16;
            float f;
            std::memcpy(&f, &u, 4);
            v[i] = f;
            break;
        }
        case DT_FP8E4M3: v[i] = fp8_to_double(p[i], true); break;
        case DT_FP8E5M2: v[i] = fp8_to_double(p[i], false); break;
        case DT_FP64: v[i] = reinterpret_cast<const double*>(p)[i]; break;
        default: throw Error(ERR_DTYPE_MISMATCH, std::string("not a float tensor: ") + dtype_name(t.dtype()));
        }
    }
    return v;
}

StoragePtr storage_from_raw_bytes(DType t, const uint8_t* bytes, size_t len, int64_t count)
{
    size_t need;
    switch (t) {
    case DT_INT4: need = static_cast<size_t>((count + 1) / 2); break;
    case DT_INT48: need = static_cast<size_t>(count) * 6; break;
    default: need = static_cast<size_t>(count) * dtype_size(t); break;
    }
    switch (t) {
    case DT_BOOL:
    case DT_INT4:
    case DT_INT8:
    case DT_INT16:
    case DT_INT32:
    case DT_INT48:
    case DT_INT64:
    case DT_SHAPE:
    case DT_FP32:
    case DT_FP16:
    case DT_BF16:
    case DT_FP8E4M3:
    case DT_FP8E5M2: break;
    default:
        throw Error(ERR_DTYPE_MISMATCH, std::string("cannot deserialize raw bytes for ") + dtype_name(t));
    }
    if (len < need)
        throw Error(ERR_DESERIALIZE, std::string(dtype_name(t)) + " tensor of " + std::to_string(count) +
                                         " elements needs " + std::to_string(need) + " bytes, got " +
                                         std::to_string(len));
    auto s = std::make_shared<Storage>();
    s->dtype = t;
    s->count = count;
    s->host.resize(s->bytes());
    uint8_t* out = s->host.data();
    if (t == DT_INT4) {
        for (int64_t i = 0; i < count; i++) {
            uint8_t nib = (bytes[i / 2] >> (4 * (i % 2))) & 0xF;
            out[i] = static_cast<uint8_t>(static_cast<int8_t>(static_cast<uint8_t>(nib << 4)) >> 4);
        }
    } else if (t == DT_INT48) {
        for (int64_t i = 0; i < count; i++) {
            uint8_t buf[8] = {0};
            std::memcpy(buf, bytes + 6 * i, 6);
            if (buf[5] & 0x80)
                buf[6] = buf[7] = 0xFF;
            std::memcpy(out + 8 * i, buf, 8);
        }
    } else if (t == DT_BOOL) {
        for (int64_t i = 0; i < count; i++)
            out[i] = bytes[i] != 0;
    } else if (need) {
        std::memcpy(out, bytes, need);
    }
    s->host_valid = true;
    return s;
}

StoragePtr storage_zeros(DType t, int64_t count)
{
    switch (t) {
    case DT_BOOL:
    case DT_INT4:
    case DT_INT8:
    case DT_INT16:
    case DT_INT32:
    case DT_INT48:
    case DT_INT64:
    case DT_SHAPE:
    case DT_FP8E4M3:
    case DT_FP8E5M2:
    case DT_FP16:
    case DT_BF16:
    case DT_FP32:
    case DT_FP64: break;
    default: throw Error(ERR_DTYPE_MISMATCH, std::string("cannot create zeros for ") + dtype_name(t));
    }
    return make_host_storage(t, count, nullptr);
}

}  // namespace tosa
