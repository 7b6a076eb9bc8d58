/*
 * tosa_mi355x.h -- C ABI of the MI355X TOSA execution path.
 *
 * The reference (emmet-horgan/tosa, `tosa-interp`, Rust) exposes this path
 * through its crate API; the entry points below are what a Rust `-sys`
 * crate (or any FFI) binds to reach the same behaviour. Each declaration
 * names the reference item it stands for. No C++ or HIP type crosses this
 * boundary: handles are opaque, shapes are int64 arrays, element types and
 * operator codes are the TOSA schema's numeric codes (schema/tosa.fbs:26-46,
 * :88-191), and every function reports errors through tosa_status plus a
 * thread-local message. Nothing here throws.
 *
 * Element storage exchanged with the host: INT4 one value per byte, INT48 as
 * int64, BOOL as uint8, FP16/BF16 as their 16-bit patterns, FP8 as bytes,
 * everything else in its natural little-endian layout.
 *
 * Threading: a tosa_graph may be shared by threads; each thread runs on its
 * own HIP stream (or the one it installed with tosa_set_stream).
 */
#ifndef TOSA_MI355X_H
#define TOSA_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error kinds: the reference's Error enum (src/error.rs:4-31), plus a device
 * error for failures of the GPU runtime itself. */
typedef enum {
    TOSA_OK = 0,
    TOSA_ERR_DESERIALIZE = 1,
    TOSA_ERR_UNSUPPORTED_OP = 2,
    TOSA_ERR_TENSOR_NOT_FOUND = 3,
    TOSA_ERR_DTYPE_MISMATCH = 4,
    TOSA_ERR_SHAPE_MISMATCH = 5,
    TOSA_ERR_BROADCAST = 6,
    TOSA_ERR_GRAPH = 7,
    TOSA_ERR_CONTROL_FLOW = 8,
    TOSA_ERR_IO = 9,
    TOSA_ERR_DEVICE = 10,
    TOSA_ERR_INVALID_ARGUMENT = 11
} tosa_status;

typedef struct tosa_graph tosa_graph;   /* an Interpreter: parsed graph + device constant cache */
typedef struct tosa_tensor tosa_tensor; /* a named, shaped, device-resident tensor */
typedef struct tosa_hook tosa_hook;     /* an InterpreterHook */

/* Message of the last error on this thread ("" if none). */
const char* tosa_last_error(void);
/* Reference Op::name() (src/ir.rs:352-457) and DType names. */
const char* tosa_op_name(uint32_t op);
const char* tosa_dtype_name(uint32_t dtype);

/* ---- graphs --------------------------------------------------------------
 * Interpreter::from_flatbuffer (src/interpreter.rs:113-116). */
tosa_status tosa_graph_from_flatbuffer(const uint8_t* data, size_t len, tosa_graph** out);
void tosa_graph_free(tosa_graph* g);
/* Interpreter::graph() (src/interpreter.rs:118-120): the main block. */
size_t tosa_graph_num_operators(const tosa_graph* g);
tosa_status tosa_graph_operator(const tosa_graph* g, size_t i, uint32_t* op, size_t* n_inputs, size_t* n_outputs);
const char* tosa_graph_operator_input(const tosa_graph* g, size_t i, size_t j);
const char* tosa_graph_operator_output(const tosa_graph* g, size_t i, size_t j);
size_t tosa_graph_num_tensors(const tosa_graph* g);
tosa_status tosa_graph_tensor(const tosa_graph* g, size_t i, const char** name, uint32_t* dtype, int32_t* shape,
                              int cap, int* rank, int* has_data);
size_t tosa_graph_num_inputs(const tosa_graph* g);
size_t tosa_graph_num_outputs(const tosa_graph* g);
const char* tosa_graph_input(const tosa_graph* g, size_t i);
const char* tosa_graph_output(const tosa_graph* g, size_t i);

/* ---- tensors (src/tensor.rs:228-250) --------------------------------------*/
/* Copies `bytes` of host data (the element storage above). */
tosa_status tosa_tensor_from_host(const char* name, const int64_t* shape, int rank, uint32_t dtype, const void* data,
                                  size_t bytes, tosa_tensor** out);
/* Wraps caller-owned device memory without copying; the memory must stay
 * valid while the tensor (or any run output sharing it) is alive. */
tosa_status tosa_tensor_from_device(const char* name, const int64_t* shape, int rank, uint32_t dtype, void* dev_ptr,
                                    size_t bytes, tosa_tensor** out);
/* Copies the elements to host memory (synchronises the stream). */
tosa_status tosa_tensor_to_host(const tosa_tensor* t, void* dst, size_t bytes);
/* Device address of the elements (uploads or recomputes them if needed). */
tosa_status tosa_tensor_device_ptr(const tosa_tensor* t, const void** ptr);
const char* tosa_tensor_name(const tosa_tensor* t);
uint32_t tosa_tensor_dtype(const tosa_tensor* t);
int tosa_tensor_rank(const tosa_tensor* t);
tosa_status tosa_tensor_shape(const tosa_tensor* t, int64_t* dims, int cap);
/* Tensor::size_bytes (src/tensor.rs:247-249): max(1, elements) * element size. */
size_t tosa_tensor_size_bytes(const tosa_tensor* t);
/* Bytes of element storage (elements * element size). */
size_t tosa_tensor_data_bytes(const tosa_tensor* t);
void tosa_tensor_free(tosa_tensor* t);

/* ---- hooks (src/stats.rs:11-298) ------------------------------------------
 * User hook: InterpreterHook's four methods as C callbacks. The tensor
 * handles passed to a callback are valid during that callback only.
 * `needs_sync`: post_op runs after the operator's kernels completed.
 * `reads_data`: the hook may read element values (disables fusion). */
typedef struct {
    void* user;
    void (*pre_op)(void* user, uint32_t op, size_t op_index, const tosa_tensor* const* inputs, size_t n_inputs);
    void (*post_op)(void* user, uint32_t op, size_t op_index, const tosa_tensor* const* inputs, size_t n_inputs,
                    const tosa_tensor* const* outputs, size_t n_outputs);
    void (*on_tensor_alloc)(void* user, const char* name, const int64_t* shape, int rank, uint32_t dtype,
                            size_t bytes);
    void (*on_tensor_free)(void* user, const char* name, size_t bytes);
    int needs_sync;
    int reads_data;
} tosa_hook_callbacks;

tosa_hook* tosa_hook_new_callbacks(const tosa_hook_callbacks* cb); /* impl InterpreterHook */
tosa_hook* tosa_hook_new_noop(void);                               /* NoopHook, stats.rs:57-58 */
tosa_hook* tosa_hook_new_stats(void);                              /* StatsCollector, stats.rs:113-195 */
tosa_hook* tosa_hook_new_flops(void);                              /* FlopCounter, stats.rs:200-263 */
tosa_hook* tosa_hook_new_trace(void);                              /* OpTrace, stats.rs:266-298 */
tosa_hook* tosa_hook_new_set(void);                                /* HookSet, stats.rs:19-76 */
/* HookSet::add; the set takes ownership of `hook`. */
tosa_status tosa_hookset_add(tosa_hook* set, tosa_hook* hook);
/* HookSet::hooks(): number and borrowed handles of the member hooks. */
size_t tosa_hookset_len(const tosa_hook* set);
tosa_hook* tosa_hookset_get(tosa_hook* set, size_t i);
void tosa_hook_free(tosa_hook* h);

/* StatsCollector fields and summary() */
uint64_t tosa_stats_total_ops(const tosa_hook* h);
size_t tosa_stats_peak_memory(const tosa_hook* h);
size_t tosa_stats_current_memory(const tosa_hook* h);
size_t tosa_stats_num_ops(const tosa_hook* h);
tosa_status tosa_stats_op(const tosa_hook* h, size_t i, const char** name, uint64_t* count, double* seconds,
                          uint64_t* elements_in, uint64_t* elements_out);
/* Writes up to cap bytes (NUL-terminated); returns the full length. */
size_t tosa_stats_summary(const tosa_hook* h, char* buf, size_t cap);
/* FlopCounter fields */
uint64_t tosa_flops_total(const tosa_hook* h);
uint64_t tosa_flops_for(const tosa_hook* h, const char* op_name);
/* OpTrace entries */
size_t tosa_trace_len(const tosa_hook* h);
tosa_status tosa_trace_entry(const tosa_hook* h, size_t i, const char** op, size_t* op_index, size_t* n_inputs,
                             size_t* n_outputs);
tosa_status tosa_trace_shape(const tosa_hook* h, size_t i, int output, size_t j, int64_t* dims, int cap, int* rank);

/* ---- running ---------------------------------------------------------------
 * Interpreter::run (src/interpreter.rs:122-147). Inputs are borrowed (their
 * handles stay the caller's); *outputs receives a new array of new handles,
 * released with tosa_outputs_free. `hook` may be NULL (NoopHook). */
tosa_status tosa_run(const tosa_graph* g, tosa_tensor* const* inputs, size_t n_inputs, tosa_hook* hook,
                     tosa_tensor*** outputs, size_t* n_outputs);
void tosa_outputs_free(tosa_tensor** outputs, size_t n);
/* Frees only the array returned by a run; the caller keeps (and later frees)
 * each tensor handle. */
void tosa_outputs_array_free(tosa_tensor** outputs);
/* run_graph / run_graph_with_stats / run_graph_with_hooks (src/lib.rs:20-43). */
tosa_status tosa_run_graph(const uint8_t* data, size_t len, tosa_tensor* const* inputs, size_t n_inputs,
                           tosa_tensor*** outputs, size_t* n_outputs);
tosa_status tosa_run_graph_with_stats(const uint8_t* data, size_t len, tosa_tensor* const* inputs, size_t n_inputs,
                                      tosa_tensor*** outputs, size_t* n_outputs, tosa_hook** stats);
tosa_status tosa_run_graph_with_hooks(const uint8_t* data, size_t len, tosa_tensor* const* inputs, size_t n_inputs,
                                      tosa_hook* hooks, tosa_tensor*** outputs, size_t* n_outputs);

/* ---- device path controls (no reference counterpart) ----------------------
 * "fusion" (default 1): fold CONV2D/DEPTHWISE_CONV2D/MATMUL -> RESCALE ->
 * CLAMP chains and quantised residual adds into single kernels.
 * "strict_float" (default 0): run float CONV2D/MATMUL in the reference's
 * sequential order (bit-exact) instead of on MFMA.
 * "deferred" (default 0): tosa_run returns once its kernels are enqueued;
 * value-dependent REQUIRE failures (RESCALE range/overflow) of such runs are
 * reported by the next tosa_synchronize. Validation errors are unaffected.
 * "conv_rows" (default 1, process-wide): int8 3x3 stride-1 CONV2D with 128
 * input channels and 17-30 pixel output rows runs on the row-tile kernel
 * (128-channel workgroups where the channels allow); 2 keeps the row-tile
 * kernel at 64-channel workgroups; 0 selects the halo kernel. All are
 * bit-exact.
 * "matmul_rows" (default 128, process-wide): rows of A per workgroup of the
 * int8 MATMUL kernel, 128 or 64; both are bit-exact. */
tosa_status tosa_set_option(const char* key, int value);
int tosa_get_option(const char* key);
/* Run this thread's work on `hip_stream` (a hipStream_t); NULL restores the
 * library's own stream. */
tosa_status tosa_set_stream(void* hip_stream);
/* Waits for this thread's stream and reports REQUIRE failures of deferred
 * runs (TOSA_ERR_GRAPH), clearing them. */
tosa_status tosa_synchronize(void);
int tosa_device_count(void);

/* ---- op-level entry points (no graph) ----------------------------------------
 * One operator on caller-owned device buffers, enqueued on `stream` (a
 * hipStream_t; NULL: this thread's stream) and returning without waiting.
 * They stand for the reference's per-operator boundary, ops::dispatch
 * (src/ops/mod.rs:22), as conformance tests and benchmarks use it.
 *
 * A RESCALE of the int32 accumulator that follows the operator in a
 * quantised graph: eval_rescale (src/ops/type_conv.rs:111-191) with
 * scale32, input zero point 0 and apply_scale_32 (src/ops/quant.rs:17-32),
 * then optionally CLAMP (src/ops/elementwise.rs:328-334). Host arrays. */
typedef struct tosa_rescale_i32 {
    const int32_t* multiplier; /* [channels], each >= 0 */
    const int8_t* shift;       /* [channels], each in [2, 62] */
    int32_t channels;          /* 1 (per tensor) or the output channels (per channel) */
    int32_t double_round;      /* 1: DOUBLE_ROUND, 0: SINGLE_ROUND */
    uint32_t output_dtype;     /* INT8, INT16 or INT32 (schema codes) */
    int32_t output_zp;         /* an int8 value for INT8 output, 0 otherwise */
    int32_t has_clamp;         /* 1: clamp the output values to [clamp_min, clamp_max] */
    int32_t clamp_min, clamp_max;
} tosa_rescale_i32;

/* int8 CONV2D: eval_conv's integer branch (src/ops/conv.rs:398-474) with
 * ConvNd::new's checks (src/ops/conv.rs:57-139). x NHWC [N,IH,IW,IC] and w
 * OHWI [OC,KH,KW,IC] int8, bias int32 [1 or OC], all device pointers (x and
 * w 16-byte aligned); pad {top, bottom, left, right}, stride {y, x},
 * dilation {y, x}. out receives NHWC [N,OH,OW,OC]: int32 without
 * `rescale`, else the rescale's output type; out_shape (may be NULL) the
 * output shape; with out NULL the call only checks its arguments and fills
 * out_shape. A value that fails apply_scale_32's range REQUIRE sets bits
 * in *device_error (a device word the caller clears and reads); with
 * device_error NULL, in the error word of this thread's stream, which the
 * next tosa_synchronize reports (then `stream` must be NULL or this thread's
 * stream). Derived data (epilogue table, packed weights) is rebuilt on every
 * call in workspace from the stream's pool. Input channels must be a
 * multiple of 16 for an unpadded 1x1 stride-1 convolution and of 64 for any
 * other (TOSA_ERR_UNSUPPORTED_OP otherwise: run such a convolution through
 * a graph). */
tosa_status tosa_conv2d_i8(const int8_t* x, const int64_t x_shape[4], const int8_t* w, const int64_t w_shape[4],
                           const int32_t* bias, int64_t bias_len, int32_t input_zp, int32_t weight_zp,
                           const int32_t pad[4], const int32_t stride[2], const int32_t dilation[2],
                           const tosa_rescale_i32* rescale, void* out, int64_t out_shape[4],
                           uint32_t* device_error, void* stream);

/* int8 MATMUL: eval_matmul's integer branch (src/ops/matmul.rs:98-153; the
 * product loop Dims::run, :80-95) with its shape checks (:112-123). a
 * [N,H,C] and b [N,C,W] int8, device pointers (16-byte aligned); a_shape
 * {N, H, C}, b_shape {N, C, W}; a_zp and b_zp int8 values. out receives
 * [N,H,W]: int32 without `rescale`, else the rescale's output type (one
 * multiplier/shift pair or W of them); out_shape (may be NULL) the output
 * shape; with out NULL the call only checks its arguments and fills
 * out_shape. device_error and stream as for tosa_conv2d_i8. The epilogue
 * table is rebuilt on every call in workspace from the stream's pool. C must
 * be a multiple of 128 and W of 16 (TOSA_ERR_UNSUPPORTED_OP otherwise: run
 * such a MATMUL through a graph). */
tosa_status tosa_matmul_i8(const int8_t* a, const int64_t a_shape[3], const int8_t* b, const int64_t b_shape[3],
                           int32_t a_zp, int32_t b_zp, const tosa_rescale_i32* rescale, void* out,
                           int64_t out_shape[3], uint32_t* device_error, void* stream);

/* No counterpart in the reference: tosa_conv2d_i8 for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). Same arguments and results, but the
 * epilogue table, packed weights and RESCALE words live in a static array of
 * 4 MiB per GPU (held until the process ends) instead of pool memory: no
 * hipMalloc, hipFree or host staging, and the RESCALE words are written by a
 * kernel from its own arguments. A call whose workspace exceeds the array is
 * rejected (TOSA_ERR_INVALID_ARGUMENT), as is a call with a RESCALE and no
 * device_error. Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams or threads) race. `stream` NULL is HIP's
 * null stream. */
tosa_status tosa_conv2d_i8_noalloc(const int8_t* x, const int64_t x_shape[4], const int8_t* w,
                                   const int64_t w_shape[4], const int32_t* bias, int64_t bias_len, int32_t input_zp,
                                   int32_t weight_zp, const int32_t pad[4], const int32_t stride[2],
                                   const int32_t dilation[2], const tosa_rescale_i32* rescale, void* out,
                                   int64_t out_shape[4], uint32_t* device_error, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TOSA_MI355X_H */
