// Device-resident tensors.
//
// The reference's TensorData is an enum of host Vecs (src/tensor.rs:6-21).
// Here a tensor's elements live in HBM; a host mirror is filled only when the
// host asks for the values (a CONST decode, an input handed over from host
// memory, an output read back). Shape and dtype always stay on the host, so
// the interpreter, its hooks and every ERROR_IF check run without touching
// the device.
//
// Element storage is the same on host and device: INT4 one value per byte,
// INT48/SHAPE as int64, BOOL as uint8, FP16/BF16 as their 16-bit patterns,
// FP8 as bytes.
//
// A *virtual* storage belongs to an intermediate that a fused kernel never
// wrote (e.g. the INT32 output of a CONV2D whose RESCALE was folded into the
// convolution). It holds a recipe that recomputes it on demand, so anyone who
// does read it still gets the reference's values.
#pragma once

#include <hip/hip_runtime_api.h>

#include <atomic>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "core.h"

namespace tosa {

struct Storage {
    DType dtype = DT_UNKNOWN;
    int64_t count = 0;  // elements

    void* dev = nullptr;
    size_t dev_bytes = 0;
    hipStream_t dev_stream = nullptr;  // allocator pool that owns `dev`
    std::atomic<bool> dev_valid{false};
    // `dev` belongs to the caller, who may rewrite it between runs: never
    // freed here, and its host mirror is re-read on every host access.
    bool external = false;
    // A graph constant shared by every run (and thread) of an Interpreter:
    // uploaded synchronously, so any stream may read it once dev_valid.
    bool shared_const = false;

    std::vector<uint8_t> host;
    std::atomic<bool> host_valid{false};

    // Upload of the host mirror issued on `ready_stream` without waiting for
    // it; another stream that reads `dev` first waits for `ready`.
    hipEvent_t ready = nullptr;
    hipStream_t ready_stream = nullptr;

    // Guards the first-use transitions (allocation, upload, download,
    // materialisation) of storages that several runs may share.
    std::recursive_mutex mu;

    // An int8 convolution's epilogue table that rules out every failure of
    // apply_scale_32's range REQUIRE (set once the table is known on the
    // host; false, i.e. check it, otherwise).
    bool scale_range_safe = false;

    // Virtual storage: fills this storage (device side) when first read.
    std::function<void(Storage&)> materialize;

    // Derived per-tensor data cached with the tensor (e.g. per-channel weight
    // sums of a convolution weight); valid as long as this storage is.
    std::shared_ptr<Storage> aux;
    int aux_kind = 0;
    // Further derived data keyed by what it was built from (e.g. the
    // epilogue table of a convolution for one bias / RESCALE combination).
    // Only immutable (graph constant) sources may be cached here.
    std::map<std::string, std::shared_ptr<Storage>> derived;

    Storage() = default;
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;
    ~Storage();

    size_t bytes() const { return static_cast<size_t>(count) * dtype_size(dtype); }
    bool is_virtual() const { return !dev_valid && !host_valid && static_cast<bool>(materialize); }

    // Device pointer with valid contents (uploads or materializes as needed).
    const void* device_in();
    // Device buffer to write all elements into; marks the device copy valid
    // and the host mirror stale.
    void* device_out();
    // Host pointer with valid contents (downloads, synchronising the stream).
    const uint8_t* host_in();
};

using StoragePtr = std::shared_ptr<Storage>;

StoragePtr make_host_storage(DType t, int64_t count, const void* data);  // copies `data`
StoragePtr make_device_storage(DType t, int64_t count);                   // uninitialised
StoragePtr wrap_device_storage(DType t, int64_t count, void* dev_ptr);    // caller-owned memory

struct Tensor {
    std::string name;
    Shape shape;
    StoragePtr data;

    DType dtype() const { return data ? data->dtype : DT_UNKNOWN; }
    int64_t len() const { return data ? data->count : 0; }
    // src/tensor.rs:243-249: element count is at least 1.
    int64_t element_count() const
    {
        int64_t n = shape_count(shape);
        return n < 1 ? 1 : n;
    }
    size_t size_bytes() const { return static_cast<size_t>(element_count()) * dtype_size(dtype()); }
};

using TensorPtr = std::shared_ptr<Tensor>;

// Host-side element access for small operands (zero points, multipliers,
// shifts, SHAPE values): every element widened to int64, or to double.
std::vector<int64_t> int_values(const Tensor& t);
std::vector<double> float_values(const Tensor& t);

// Decode serialized (little-endian) tensor data: src/tensor.rs:86-167.
// INT4 packs two per byte (low nibble first), INT48 uses 6 bytes.
StoragePtr storage_from_raw_bytes(DType t, const uint8_t* bytes, size_t len, int64_t count);
StoragePtr storage_zeros(DType t, int64_t count);  // src/tensor.rs:63-80

}  // namespace tosa
