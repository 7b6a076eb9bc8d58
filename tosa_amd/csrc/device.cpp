#include "device.h"

#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace tosa {

void hip_check(hipError_t e, const char* what)
{
    if (e != hipSuccess)
        throw Error(ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

std::string device_error_message(uint32_t bits)
{
    std::string m;
    if (bits & DERR_SCALE_PARAMS)
        m += "apply_scale: invalid multiplier or shift; ";
    if (bits & DERR_SCALE_RANGE)
        m += "apply_scale_32: value out of range for shift; ";
    if (bits & DERR_SCALE_RESULT)
        m += "apply_scale: result exceeds int32; ";
    if (bits & DERR_RESCALE_I32)
        m += "RESCALE: result exceeds the int32 range; ";
    if (!m.empty())
        m.resize(m.size() - 2);
    return m;
}

namespace {

struct Pools {
    std::mutex mu;
    // stream -> (size -> free blocks)
    std::unordered_map<hipStream_t, std::multimap<size_t, void*>> free;
    size_t cached = 0;
};

Pools& pools()
{
    static Pools* p = new Pools();  // never destroyed: blocks may be freed during exit
    return *p;
}

size_t round_size(size_t b)
{
    if (b <= 256)
        return 256;
    if (b <= (1u << 20)) {  // next power of two up to 1 MiB
        size_t r = 512;
        while (r < b)
            r <<= 1;
        return r;
    }
    const size_t g = 2u << 20;  // 2 MiB granules above
    return (b + g - 1) / g * g;
}

struct PinnedBlock {
    void* p = nullptr;
    size_t bytes = 0;
    hipEvent_t ev = nullptr;  // recorded after the copy out of the block
    bool held = false;        // acquired and not yet released
};

struct PinnedPool {
    std::mutex mu;
    std::vector<PinnedBlock> idle, busy;
    size_t idle_bytes = 0;
};

PinnedPool& pinned_pool()
{
    static PinnedPool* p = new PinnedPool();  // never destroyed, like the device pools
    return *p;
}

// Blocks kept for reuse beyond this many bytes go back to the driver.
constexpr size_t PINNED_KEEP_BYTES = size_t(1) << 30;

thread_local Stream* t_stream = nullptr;
thread_local hipStream_t t_user_stream = nullptr;

std::mutex g_err_mu;
struct ErrWord {
    uint32_t* dev = nullptr;
    uint32_t* host = nullptr;
};
std::unordered_map<hipStream_t, ErrWord> g_err_words;

// The device error word of stream `s` and the pinned host word it is read
// back into (a copy into pageable memory takes the runtime's staged path,
// about twice the round trip of one into pinned memory).
ErrWord error_word_for(hipStream_t s)
{
    std::lock_guard<std::mutex> lk(g_err_mu);
    auto it = g_err_words.find(s);
    if (it != g_err_words.end())
        return it->second;
    ErrWord w;
    void* p = nullptr;
    hip_check(hipMalloc(&p, 256), "hipMalloc(error word)");
    hip_check(hipMemset(p, 0, 256), "hipMemset(error word)");
    w.dev = static_cast<uint32_t*>(p);
    void* h = nullptr;
    hip_check(hipHostMalloc(&h, 64, hipHostMallocDefault), "hipHostMalloc(error word)");
    w.host = static_cast<uint32_t*>(h);
    *w.host = 0;
    g_err_words[s] = w;
    return w;
}

}  // namespace

int device_count()
{
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess)
        return 0;
    return n;
}

bool device_available() { return device_count() > 0; }

Stream& thread_stream()
{
    if (t_user_stream) {
        static thread_local Stream user;
        if (user.s != t_user_stream) {
            user.s = t_user_stream;
            const ErrWord w = error_word_for(t_user_stream);
            user.err = w.dev;
            user.err_host = w.host;
        }
        return user;
    }
    if (!t_stream) {
        if (!device_available())
            throw Error(ERR_DEVICE, "no HIP device is available (the MI355X path needs a GPU)");
        Stream* st = new Stream();
        hip_check(hipStreamCreateWithFlags(&st->s, hipStreamNonBlocking), "hipStreamCreate");
        const ErrWord w = error_word_for(st->s);
        st->err = w.dev;
        st->err_host = w.host;
        t_stream = st;
    }
    return *t_stream;
}

void set_thread_stream(hipStream_t s) { t_user_stream = s; }

void* dev_alloc(size_t bytes, hipStream_t s)
{
    size_t r = round_size(bytes);
    Pools& P = pools();
    {
        std::lock_guard<std::mutex> lk(P.mu);
        auto& m = P.free[s];
        auto it = m.find(r);
        if (it != m.end()) {
            void* p = it->second;
            m.erase(it);
            P.cached -= r;
            return p;
        }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, r);
    if (e == hipErrorOutOfMemory) {
        // Return every cached block to the driver and try once more.
        std::lock_guard<std::mutex> lk(P.mu);
        (void)hipDeviceSynchronize();
        for (auto& [st, m] : P.free)
            for (auto& [sz, q] : m)
                (void)hipFree(q);
        P.free.clear();
        P.cached = 0;
        e = hipMalloc(&p, r);
    }
    hip_check(e, "hipMalloc");
    return p;
}

void dev_free(void* p, size_t bytes, hipStream_t s)
{
    if (!p)
        return;
    size_t r = round_size(bytes);
    Pools& P = pools();
    std::lock_guard<std::mutex> lk(P.mu);
    P.free[s].emplace(r, p);
    P.cached += r;
}

void* pinned_acquire(size_t bytes)
{
    const size_t r = round_size(bytes ? bytes : 1);
    PinnedPool& P = pinned_pool();
    {
        std::lock_guard<std::mutex> lk(P.mu);
        // Blocks whose copies have run become idle.
        for (size_t i = 0; i < P.busy.size();) {
            if (!P.busy[i].held && hipEventQuery(P.busy[i].ev) == hipSuccess) {
                P.idle_bytes += P.busy[i].bytes;
                P.idle.push_back(P.busy[i]);
                P.busy[i] = P.busy.back();
                P.busy.pop_back();
            } else {
                i++;
            }
        }
        size_t best = P.idle.size();
        for (size_t i = 0; i < P.idle.size(); i++)
            if (P.idle[i].bytes >= r && (best == P.idle.size() || P.idle[i].bytes < P.idle[best].bytes))
                best = i;
        if (best < P.idle.size()) {
            PinnedBlock b = P.idle[best];
            P.idle[best] = P.idle.back();
            P.idle.pop_back();
            P.idle_bytes -= b.bytes;
            b.held = true;  // the caller's until pinned_release
            P.busy.push_back(b);
            return b.p;
        }
        while (P.idle_bytes + r > PINNED_KEEP_BYTES && !P.idle.empty()) {
            (void)hipHostFree(P.idle.back().p);
            if (P.idle.back().ev)
                (void)hipEventDestroy(P.idle.back().ev);
            P.idle_bytes -= P.idle.back().bytes;
            P.idle.pop_back();
        }
    }
    PinnedBlock b;
    hip_check(hipHostMalloc(&b.p, r, hipHostMallocDefault), "hipHostMalloc(staging)");
    b.bytes = r;
    b.held = true;
    hip_check(hipEventCreateWithFlags(&b.ev, hipEventDisableTiming), "hipEventCreate(staging)");
    std::lock_guard<std::mutex> lk(P.mu);
    P.busy.push_back(b);
    return b.p;
}

void pinned_release(void* p, hipStream_t s)
{
    PinnedPool& P = pinned_pool();
    std::lock_guard<std::mutex> lk(P.mu);
    for (auto& b : P.busy)
        if (b.p == p && b.held) {
            // The block stays busy until everything enqueued on `s` so far
            // has run.
            b.held = false;
            hip_check(hipEventRecord(b.ev, s), "hipEventRecord(staging)");
            return;
        }
}

size_t dev_cached_bytes()
{
    Pools& P = pools();
    std::lock_guard<std::mutex> lk(P.mu);
    return P.cached;
}

uint32_t* stream_error_word(hipStream_t s) { return error_word_for(s).dev; }

void clear_error_word(Stream& st) { hip_check(hipMemsetAsync(st.err, 0, sizeof(uint32_t), st.s), "clear error word"); }

uint32_t read_error_word(Stream& st)
{
    hip_check(hipMemcpyAsync(st.err_host, st.err, sizeof(uint32_t), hipMemcpyDeviceToHost, st.s), "read error word");
    hip_check(hipStreamSynchronize(st.s), "hipStreamSynchronize");
    return *static_cast<volatile uint32_t*>(st.err_host);
}

}  // namespace tosa
