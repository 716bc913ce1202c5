/*
 * xs_hip.h -- the C-ABI of the MI355X (gfx950) device for xpu-serve's elementwise, broadcast and reduction ops.
 *
 * Each entry point replaces one launcher of the reference's device-dispatch surface, `xs::sycl_be::*` in
 * src/backend/sycl/sycl_kernels.h, with a plain-C function:
 *   - `sycl::queue&` becomes an opaque stream handle (`void*`, a hipStream_t; NULL is the null stream);
 *   - template parameters (X, Y, CT, I) become `xs_dtype` arguments whose values are the reference's `DType`
 *     enumerators (src/tensor/dtype.h:17);
 *   - the reference's C++ exceptions (`xs::Error`, src/util/error.h:12-35) become an `int` status: XS_HIP_OK, or a
 *     code whose message `xs_hip_last_error()` returns (thread-local, naming the op and what is wrong).
 * Every launcher enqueues on the stream and returns without waiting, as the reference's do (sycl_kernels.h:3).
 * Pointers are device pointers; sizes and strides are element counts (int64). No torch, SYCL or HIP types appear here.
 *
 * Numerical contract (checked by the repository's parity tests against the reference's CPU path, cpu-ref):
 * f32 outputs within 1e-5 relative, f16/bf16 outputs within one unit in the last place of the output dtype (inputs
 * widened exactly, arithmetic in f32 or f64), argmax indices, int8 codes and scales bit-exact.
 */
#ifndef XS_HIP_H
#define XS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Status, errors, version -------------------------------------------------------------------------------- */

enum {
    XS_HIP_OK = 0,
    XS_HIP_EINVAL = 1,       /* a bad argument: shape, dtype, pointer, alignment or option */
    XS_HIP_EUNSUPPORTED = 2, /* a valid request this device does not implement (e.g. a TurboQuant KV format) */
    XS_HIP_ERUNTIME = 3      /* the HIP runtime refused a launch or a memory operation */
};

/* The message of the calling thread's last failed call ("" when none failed). Replaces the text of the xs::Error the
 * reference throws (src/util/error.h:25-28). */
const char* xs_hip_last_error(void);
/* 1 for this version of the ABI. */
int xs_hip_abi_version(void);

/* ---- Types --------------------------------------------------------------------------------------------------- */

/* Values of the reference's `enum class DType : uint8_t` (src/tensor/dtype.h:17), in its order. The kernels accept
 * F32, F16, BF16 for floats, I32 and I64 for positions, I8 for KV codes. */
typedef enum {
    XS_F32 = 0,
    XS_F16 = 1,
    XS_BF16 = 2,
    XS_I64 = 3,
    XS_I32 = 4,
    XS_I8 = 5,
    XS_U8 = 6,
    XS_BOOL = 7
} xs_dtype;

/* `xs::sycl_be::UnaryOp` (src/backend/sycl/sycl_kernels.h:21), in its order. The act_* entry points take SILU,
 * GELU_TANH, SIGMOID and GELU. */
typedef enum {
    XS_UNARY_SCALE = 0,
    XS_UNARY_TANH = 1,
    XS_UNARY_GELU_TANH = 2,
    XS_UNARY_SOFTCAP = 3,
    XS_UNARY_SIGMOID = 4,
    XS_UNARY_SILU = 5,
    XS_UNARY_SOFTPLUS = 6,
    XS_UNARY_CLAMP = 7,
    XS_UNARY_GELU = 8
} xs_unary_op;

/* `xs::sycl_be::BinaryOp` (sycl_kernels.h:34). */
typedef enum { XS_BINARY_ADD = 0, XS_BINARY_MUL = 1, XS_BINARY_DIV = 2 } xs_binary_op;

/* `xs::quant::KvFormat` (src/quant/kv_format.h:11-17). xs_hip_quantize_kv / xs_hip_dequantize_kv take XS_KV_I8 and
 * the TurboQuant formats, read by xs_hip_attention_i8 and xs_hip_attention_quantized; the Float format's rows are
 * written by xs_hip_kv_store_pair and read by xs_hip_attention. */
typedef enum { XS_KV_FLOAT = 0, XS_KV_I8 = 1, XS_KV_TURBO4 = 2, XS_KV_TURBO3 = 3, XS_KV_TURBO2 = 4 } xs_kv_format;

/* numpy broadcasting over at most XS_MAX_RANK dims: the out shape and the element strides of a, b and y per out dim.
 * A stride of 0 is a broadcast dim; any other stride (including a column slice's row stride) is honoured. Replaces
 * `xs::sycl_be::Broadcast` (sycl_kernels.h:37-42), which has no y strides (its y is always contiguous: pass the
 * row-major strides of `out`, or let xs_hip_broadcast_fill set them). */
#define XS_MAX_RANK 6
typedef struct {
    int32_t rank;
    int64_t out[XS_MAX_RANK];
    int64_t stride_a[XS_MAX_RANK];
    int64_t stride_b[XS_MAX_RANK];
    int64_t stride_y[XS_MAX_RANK];
} xs_broadcast;

/* Fills `bc` for row-major contiguous a [a_rank dims] and b [b_rank dims] broadcast like numpy (shapes right-aligned,
 * a dim of 1 stretches) into a contiguous y: the host half of cpu_ref::broadcast_shape / broadcast_strides
 * (src/backend/cpu_ref/ops.cpp:42-66). Fails (XS_HIP_EINVAL) on shapes that do not broadcast. */
int xs_hip_broadcast_fill(xs_broadcast* bc, const int64_t* a_shape, int32_t a_rank, const int64_t* b_shape,
                          int32_t b_rank);

/* ---- Device, memory, streams, events (the session's plumbing: sycl_backend.cpp:64-107 DeviceBuffer) ---------- */

int xs_hip_device_count(int* count);
/* name: at least 256 bytes. */
int xs_hip_device_info(int device, char* name, size_t name_len, uint64_t* memory_bytes, int* compute_units);
int xs_hip_set_device(int device);
int xs_hip_malloc(void** ptr, size_t bytes);
int xs_hip_free(void* ptr);
int xs_hip_memset(void* ptr, int value, size_t bytes, void* stream);
int xs_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream); /* synchronous w.r.t. the host */
int xs_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream); /* synchronous w.r.t. the host */
int xs_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream); /* asynchronous */
/* Asynchronous host copies, for host memory from xs_hip_host_alloc (page-locked): the host memory must stay as it is
 * until the stream has finished the copy. */
int xs_hip_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream);
int xs_hip_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream);
int xs_hip_host_alloc(void** ptr, size_t bytes);
int xs_hip_host_free(void* ptr);
int xs_hip_stream_create(void** stream);
int xs_hip_stream_destroy(void* stream);
int xs_hip_stream_synchronize(void* stream);
int xs_hip_device_synchronize(void);
int xs_hip_event_create(void** event);
int xs_hip_event_destroy(void* event);
int xs_hip_event_record(void* event, void* stream);
/* Milliseconds between two recorded events (waits for `end`). */
int xs_hip_event_elapsed_ms(float* ms, void* start, void* end);
/* Stream capture into a HIP graph (relaxed capture mode): begin, launch the calls to record, end -> an executable
 * graph; replay it with xs_hip_graph_launch; free it with xs_hip_graph_destroy. The launchers above record no memset
 * or allocation, so any sequence of them can be captured. */
int xs_hip_stream_begin_capture(void* stream);
int xs_hip_stream_end_capture(void* stream, void** graph_exec);
int xs_hip_graph_launch(void* graph_exec, void* stream);
int xs_hip_graph_destroy(void* graph_exec);

/* ---- Elementwise and broadcast ------------------------------------------------------------------------------- */

/* y = a op b under `bc` (any strides), a/b/y each F32, F16 or BF16; arithmetic in f32 on exactly widened operands,
 * rounded once to y's dtype. Replaces sycl_be::binary (sycl_kernels.h:43-44); semantics cpu_ref::add / mul / div
 * (ops.cpp:68-93, 201-207, 401-403). In-place (y == a or y == b with the same strides) is allowed. */
int xs_hip_binary(void* stream, xs_binary_op op, xs_dtype a_dtype, const void* a, xs_dtype b_dtype, const void* b,
                  xs_dtype y_dtype, void* y, const xs_broadcast* bc);
/* Contiguous fast paths: same shape (sycl_kernels.h:46-47) and b repeating every `period` elements of a, a row vector
 * over the leading dims (sycl_kernels.h:48-49). n % period == 0. */
int xs_hip_binary_same(void* stream, xs_binary_op op, xs_dtype dtype, const void* a, const void* b, xs_dtype y_dtype,
                       void* y, int64_t n);
int xs_hip_binary_period(void* stream, xs_binary_op op, xs_dtype dtype, const void* a, const void* b,
                         xs_dtype y_dtype, void* y, int64_t n, int64_t period);
/* Fused residuals (sycl_kernels.h:51-55), f32 in: y = a + b * c[i % period] and y = a + (b + c[i % period]); the
 * result equals the two unfused f32 ops cpu-ref evaluates in graph order. */
int xs_hip_add_mul(void* stream, const float* a, const float* b, const float* c, xs_dtype y_dtype, void* y, int64_t n,
                   int64_t period);
int xs_hip_add3(void* stream, const float* a, const float* b, const float* c, xs_dtype y_dtype, void* y, int64_t n,
                int64_t period);

/* y = op(x), n elements, x and y F32, F16 or BF16: Scale (y = x * a), Tanh, GeluTanh, Softcap (y = a tanh(x / a)),
 * Sigmoid, Silu, Softplus (identity above 20), Clamp (min(max(x, a), b), NaN kept), Gelu. Replaces sycl_be::unary
 * (sycl_kernels.h:21-25), whose x is f32; semantics cpu_ref::scale ... clamp (ops.cpp:209-258): Scale and Clamp
 * exactly as cpu-ref's f32 arithmetic, the GELUs in f64 as cpu-ref, Tanh / Softcap / Softplus / Sigmoid / Silu with
 * f32 transcendentals (within 1e-5 relative of cpu-ref's f64 for f32 outputs, within one unit of a 16-bit output). */
int xs_hip_unary(void* stream, xs_unary_op op, xs_dtype x_dtype, const void* x, xs_dtype y_dtype, void* y, int64_t n,
                 float a, float b);
/* y = act(x) * b, same shapes, x/b in x_dtype (F32, F16, BF16), y in y_dtype; act is SILU, GELU_TANH, SIGMOID or
 * GELU. Replaces sycl_be::act_mul (sycl_kernels.h:28-29), the fused Mul(Silu(gate), up) of gated_mlp
 * (src/models/common/blocks.cpp:23-27); semantics cpu_ref::silu etc. then cpu_ref::mul (ops.cpp:201-247). */
int xs_hip_act_mul(void* stream, xs_unary_op act, xs_dtype x_dtype, const void* x, const void* b, xs_dtype y_dtype,
                   void* y, int64_t n);
/* y = act(x + bias[i % period]), x f32. Replaces sycl_be::unary_bias (sycl_kernels.h:31-32). */
int xs_hip_unary_bias(void* stream, xs_unary_op act, const float* x, const float* bias, xs_dtype y_dtype, void* y,
                      int64_t n, int64_t period);
/* The gated MLP activation on 2-D operands with row strides (column slices of a fused gate|up buffer allowed):
 * y[r, c] = act(x[r, c] + bias[c]) * b[r, c] for r < rows, c < cols; bias may be NULL. x, b, bias in x_dtype.
 * One kernel for what the reference launches as unary_bias then act_mul (sycl_backend.cpp:1004-1047, 1899-1907);
 * the value equals cpu-ref's Add, Silu, Mul in f32 (ops.cpp:201-247) rounded to y_dtype. */
int xs_hip_act_bias_mul_2d(void* stream, xs_unary_op act, xs_dtype x_dtype, const void* x, int64_t x_row_stride,
                           const void* b, int64_t b_row_stride, const void* bias, xs_dtype y_dtype, void* y,
                           int64_t y_row_stride, int64_t rows, int64_t cols);
/* y = x converted to y_dtype (F32/F16/BF16 both ways): round to nearest even, f16 overflow to inf, NaN stays NaN
 * (src/util/half.h:19-25, half.cpp:36-56). Replaces sycl_be::to_half (sycl_kernels.h:130). */
int xs_hip_convert(void* stream, xs_dtype x_dtype, const void* x, xs_dtype y_dtype, void* y, int64_t n);

/* ---- Row reductions ------------------------------------------------------------------------------------------ */

/* Rows of `width`: y = x / rms(x) [* w] [+ bias], w and bias f32 [width] or NULL, the mean of squares in f32 and then
 * f64, eps added in f64. x f32, F16 or BF16; y F32, F16 or BF16. Replaces sycl_be::rms_norm (sycl_kernels.h:88-90);
 * semantics cpu_ref::rms_norm (ops.cpp:260-281). */
int xs_hip_rms_norm(void* stream, xs_dtype x_dtype, const void* x, const float* w, const float* bias, xs_dtype y_dtype,
                    void* y, int64_t rows, int64_t width, float eps);
/* The residual stream's add-and-norm in one pass: h = x + residual (f32, exact as cpu_ref::add), h_out = h (may be
 * `residual` or `x` itself, in place), y = rms_norm(h) [* w] [+ bias]. The graph pattern
 * h = add(h, f(rms_norm(h))) (src/models/qwen3/qwen3_decoder.cpp:101-102) evaluated by cpu-ref as Add then RmsNorm. */
int xs_hip_add_rms_norm(void* stream, const float* x, const float* residual, const float* w, const float* bias,
                        float* h_out, xs_dtype y_dtype, void* y, int64_t rows, int64_t width, float eps);
/* Rows of `width`: y = (h - mean(h)) / sqrt(var(h) + eps) [* w] [+ b], h = x + shift (shift f32 [width], added in f32,
 * or NULL: h = x); w and b f32 [width] or NULL. Mean and variance in f64, output formed in f64 and rounded once. x
 * F32, F16 or BF16; y F32, F16 or BF16. Replaces sycl_be::layer_norm (sycl_kernels.h:91-94); semantics
 * cpu_ref::layer_norm (ops.cpp:595-614), after cpu_ref::add for the shift. */
int xs_hip_layer_norm(void* stream, xs_dtype x_dtype, const void* x, const float* shift, const float* w, const float* b,
                      xs_dtype y_dtype, void* y, int64_t rows, int64_t width, float eps);
/* Rows of `width`, f32: y = x * min(1, threshold / (|x| + eps)), |x| the row's L2 norm in f64. Replaces
 * sycl_be::l2_clip (sycl_kernels.h:141-142); semantics cpu_ref::l2_clip (ops.cpp:401-412). */
int xs_hip_l2_clip(void* stream, const float* x, float* y, int64_t rows, int64_t width, float threshold, float eps);
/* y [outer, inner] = the sum over the middle axis of x [outer, dim, inner], f32, accumulated in f64. Replaces
 * sycl_be::reduce_sum (sycl_kernels.h:80-81); semantics cpu_ref::reduce_sum (ops.cpp:686-705). */
int xs_hip_reduce_sum(void* stream, const float* x, float* y, int64_t outer, int64_t dim, int64_t inner);
/* Row softmax, f32, rows of `width`. Replaces sycl_be::softmax (sycl_kernels.h:58); semantics cpu_ref::softmax
 * (ops.cpp:644-661): max, sum of exp, exp / sum. */
int xs_hip_softmax(void* stream, const float* x, float* y, int64_t rows, int64_t width);
/* The masked attention-score form: per row r, s = fl32(x * scale) for keys c < valid_len[r] (or `valid_len_all` when
 * valid_len is NULL) and -inf beyond, then softmax; masked keys come out exactly 0. x/y rows `row_stride` apart.
 * Equals cpu-ref's Scale (ops.cpp:209-211), Add of a 0/-inf mask, Softmax (ops.cpp:644-661).
 * With `scratch` (xs_hip_softmax_scratch bytes, 16-byte aligned), a few wide rows are split over several workgroups of
 * one launch that pass each chunk's (max, sum) through it; with NULL each row is one workgroup. The scratch must be
 * zero-filled before its first use; every call leaves it ready for the next, so one buffer (of the largest size
 * asked for) serves any sequence of calls of any shapes on one stream. Concurrent calls must not share one scratch. */
int xs_hip_softmax_masked(void* stream, const float* x, float* y, int64_t rows, int64_t width, int64_t row_stride,
                          float scale, const int64_t* valid_len, int64_t valid_len_all, void* scratch);
/* Bytes of scratch xs_hip_softmax_masked can use for rows of `width` (0: it would not split them). No reference
 * counterpart (cpu-ref's softmax needs none). */
size_t xs_hip_softmax_scratch(int64_t rows, int64_t width);
/* Polls a workgroup of a split launch (xs_hip_softmax_masked) makes for its row's other chunks before it computes the
 * row's partials alone (same result, slower); 0 takes that path at once. A testing hook with no reference
 * counterpart: the fallback keeps every launch finite when the chip cannot hold a split launch's workgroups at once. */
void xs_hip_set_spin_limit(int polls);
/* Bytes of scratch xs_hip_topk needs (0: none, NULL allowed). Replaces sycl_be::topk_scratch (sycl_kernels.h:61). */
size_t xs_hip_topk_scratch(int64_t rows, int64_t width, int64_t k);
/* The k largest per row of x [rows, width] f32: values f32 and indices i32 [rows, k], largest first, equal values keep
 * the lower index first (cpu_ref::topk, ops.cpp:663-684; spec graph.h:70-71). k = 1 is argmax (blocks::argmax_rows,
 * blocks.cpp:36-38). `scratch` (8-byte aligned, any contents) holds xs_hip_topk_scratch bytes: for k = 1 the per-chunk
 * partials of wide rows, for 1 < k <= 1024 on rows wider than 4096 each 4096-value chunk's threshold bin, candidate
 * count and candidates (room for max(256, 4k) words); concurrent calls must not share one. Replaces sycl_be::topk
 * (sycl_kernels.h:62-63). */
int xs_hip_topk(void* stream, const float* x, float* values, int32_t* indices, int64_t rows, int64_t width, int64_t k,
                void* scratch);
/* Bytes of zero-filled scratch xs_hip_argmax needs (0: none, NULL allowed). No reference counterpart. */
size_t xs_hip_argmax_scratch(int64_t rows, int64_t width);
/* Argmax per row of x [rows, width] f32 in one launch: values f32 [rows] the row's maximum, indices i32 [rows] its
 * lowest index among exact ties; NaN is never picked, and a row of nothing but NaN reports index 0 and x[0] -- the
 * results of xs_hip_topk with k = 1 (cpu_ref::topk, ops.cpp:663-684; blocks::argmax_rows, blocks.cpp:36-38). An
 * extension of this device: the reference's argmax is sycl_be::topk with k = 1 (sycl_kernels.h:62-63), two launches
 * through its scratch. `scratch` (xs_hip_argmax_scratch bytes, 8-byte aligned) must be zero-filled before its first
 * use; every call leaves it zero-filled again, so one buffer (of the largest size asked for) serves any sequence of
 * calls of any shapes on one stream. Concurrent calls must not share one scratch. */
int xs_hip_argmax(void* stream, const float* x, float* values, int32_t* indices, int64_t rows, int64_t width,
                  void* scratch);

/* ---- RoPE ---------------------------------------------------------------------------------------------------- */

/* Rotate-half (NeoX) RoPE of x [tokens, heads, dim] into y (y may be x). positions [tokens] or [tokens, sections]
 * (pos_dtype I32 or I64), inv_freq f32 [rotary / (2 sections)] (or [rotary / 2] with pair_axes); rotary 0 = dim;
 * channels past `rotary` pass through. With pair_axes (i32 [rotary / 2], device) one section whose pair i reads
 * positions[:, pair_axes[i]]. Angles pos * inv_freq and their cos/sin in f64, rotation in f64, rounded to f32 and then
 * to y's dtype -- cpu_ref::rope (ops.cpp:343-399). Replaces sycl_be::rope (sycl_kernels.h:114-116). */
int xs_hip_rope(void* stream, xs_dtype x_dtype, const void* x, xs_dtype pos_dtype, const void* positions,
                const float* inv_freq, xs_dtype y_dtype, void* y, int64_t tokens, int64_t heads, int64_t dim,
                int64_t rotary, int64_t sections, const int32_t* pair_axes);

/* RoPE of two tensors of the same tokens in one launch -- the Q and K of a step, which share positions and inv_freq:
 * xa/ya [tokens, heads_a, dim] and xb/yb [tokens, heads_b, dim], same dtypes; each rotated exactly as xs_hip_rope
 * rotates it (each y may be its x). One launch computes each (token, pair) angle once for both tensors' heads. No
 * reference counterpart: the reference launches rope once per tensor (sycl_backend.cpp:2187-2206). */
int xs_hip_rope2(void* stream, xs_dtype x_dtype, const void* xa, void* ya, int64_t heads_a, const void* xb, void* yb,
                 int64_t heads_b, xs_dtype pos_dtype, const void* positions, const float* inv_freq, xs_dtype y_dtype,
                 int64_t tokens, int64_t dim, int64_t rotary, int64_t sections, const int32_t* pair_axes);

/* ---- int8 KV cache ------------------------------------------------------------------------------------------- */

/* Codes and scales of x [rows, width] (x_dtype F32, F16 or BF16), by format. Replaces sycl_be::quantize_kv
 * (sycl_kernels.h:213-214).
 * XS_KV_I8: per row amax = max |x|, inv = 127 / amax (f32, correctly rounded; 0 for an all-zero row),
 *   code = clamp(round-half-even(x * inv), -127, 127), scale = amax / 127; codes int8 [rows, width], scales f32 [rows]
 *   (kv_row_bytes I8, src/quant/kv_format.cpp:47-48); semantics quant::quantize_kv_row_i8 (src/quant/quant.cpp:259-267).
 * XS_KV_TURBO4 / TURBO3 / TURBO2: width a multiple of 128; each group of 128 values rotated (sign flips, Walsh-Hadamard,
 *   sign flips) and each coordinate rounded to the nearest of 16 / 8 / 4 centroids; codes [rows * width / 128,
 *   16 * bits] bytes in the group layout of kv_turbo.h:84-87 and `scales` as f16 norms [rows * width / 128] (2-byte
 *   aligned); the same bits as quant::turbo::quantize_group (src/quant/kv_turbo.cpp:47-84). x 16-byte aligned. */
int xs_hip_quantize_kv(void* stream, xs_kv_format format, xs_dtype x_dtype, const void* x, void* codes, void* scales,
                       int64_t rows, int64_t width);
/* out [rows, width] (F32, F16 or BF16) = the values the codes store, rounded to out's dtype. Replaces
 * sycl_be::dequantize_kv (sycl_kernels.h:217-218). XS_KV_I8: fl32(code * scale[row]), quant::round_trip_kv_i8
 * (quant.cpp:269-277). TurboQuant: centroid(code) * norm per group, still rotated (quant::turbo::decode_group,
 * kv_turbo.cpp:86-91; xs_hip_kv_rotate rotates back); out 16-byte aligned. */
int xs_hip_dequantize_kv(void* stream, xs_kv_format format, const void* codes, const void* scales, xs_dtype out_dtype,
                         void* out, int64_t rows, int64_t width);
/* No counterpart in the reference: for callers that capture a step into a HIP graph and replay it while the cache
 * grows. The XS_KV_I8 quantize of `rows` rows, written at rows row0[0] * rows_per_unit + r of a cache of
 * `capacity_rows` rows (codes int8 [capacity_rows, width], scales f32 [capacity_rows]); row0 is a device int64 read
 * when the kernel runs, so one captured launch appends wherever the cache ends at replay. A destination outside the
 * cache writes nothing. */
int xs_hip_quantize_kv_at(void* stream, xs_dtype x_dtype, const void* x, void* codes, void* scales, int64_t rows,
                          int64_t width, const int64_t* row0, int64_t rows_per_unit, int64_t capacity_rows);
/* No counterpart in the reference, as xs_hip_quantize_kv_at: the TurboQuant quantize (format XS_KV_TURBO4, 3 or 2) of
 * `rows` rows, written at rows row0[0] * rows_per_unit + r of a cache of `capacity_rows` rows (codes
 * [capacity_rows * width / 128, 16 * bits] bytes, f16 norms [capacity_rows * width / 128]); a destination outside the
 * cache writes nothing. */
int xs_hip_quantize_kv_turbo_at(void* stream, xs_kv_format format, xs_dtype x_dtype, const void* x, void* codes,
                                void* norms, int64_t rows, int64_t width, const int64_t* row0, int64_t rows_per_unit,
                                int64_t capacity_rows);
/* No counterpart in the reference (it appends keys and values by two launches): the XS_KV_I8 quantize of a step's
 * keys k and values v, both [rows, width] of x_dtype, in one launch, into their own caches -- at rows [0, rows) of
 * k_codes / k_scales and v_codes / v_scales with row0 NULL, or at the device-held row as xs_hip_quantize_kv_at. The
 * bits are xs_hip_quantize_kv's for each. */
int xs_hip_quantize_kv_pair(void* stream, xs_dtype x_dtype, const void* k, const void* v, void* k_codes, void* k_scales,
                            void* v_codes, void* v_scales, int64_t rows, int64_t width, const int64_t* row0,
                            int64_t rows_per_unit, int64_t capacity_rows);

/* The Float KV format's append: a step's keys k and values v, both [rows, width] of x_dtype (f32, f16 or bf16), stored
 * as rows of row_dtype (XS_F16 at f16 precision, XS_F32 at f32; RNE) -- at rows [0, rows) of k_rows / v_rows with row0
 * NULL, or at row row0[0] * rows_per_unit of caches of capacity_rows rows, read from device memory when the kernel runs
 * (rows past the capacity are written nowhere); v and v_rows both NULL append keys only. Replaces the SYCL session's
 * float append (sycl_backend.cpp:2224-2231: to_half, or a copy at f32) in one launch for keys and values. */
int xs_hip_kv_store_pair(void* stream, xs_dtype x_dtype, const void* k, const void* v, xs_dtype row_dtype,
                         void* k_rows, void* v_rows, int64_t rows, int64_t width, const int64_t* row0,
                         int64_t rows_per_unit, int64_t capacity_rows);

/* y [rows, width] = x with each group of 128 values rotated as the TurboQuant formats rotate a row (inverse = 0), or
 * rotated back (inverse = 1); f32, 16-byte aligned, y may be x. Replaces sycl_be::kv_rotate (sycl_kernels.h:219-221);
 * semantics quant::turbo::rotate_group (kv_turbo.cpp:118-129). */
int xs_hip_kv_rotate(void* stream, const float* x, float* y, int64_t rows, int64_t width, int inverse);

/* ---- Attention over the int8 KV cache ------------------------------------------------------------------------ */

/* Decode attention reading the int8 cache in place: q f32 [tokens, q_heads, head_dim]; keys and values as
 * xs_hip_quantize_kv writes them, codes int8 [kv_len, kv_heads, head_dim] and scales f32 [kv_len, kv_heads]; out f32
 * [tokens, q_heads, head_dim]. Query head h reads KV head h / (q_heads / kv_heads). Query t sits at position
 * kv_len - tokens + t; causal: keys up to it; window > 0: keys within window - 1 of it (both sides when not causal);
 * otherwise every key. s = scale * q . k (softcap > 0: softcap * tanh(s / softcap)), softmax, weighted sum of the
 * values fl32(code * scale) -- cpu_ref::attention over the values the int8 cache stores (ops.cpp:113-156, 535-594;
 * quant.cpp:269-277), to the reference's device tolerance for a quantized cache (device_attention.cpp:23-27: f32
 * atol 1e-4, rtol 1e-4). head_dim 64, 128 or 256; 1 to 8 query heads per KV head; q, out, codes 16-byte aligned.
 * `split` > 1 divides each query's keys over that many waves (flash decoding) and needs
 * xs_hip_attention_i8_scratch bytes of `scratch` (16-byte aligned) for their partial rows; xs_hip_attention_i8_split
 * suggests a split that fills the device. Replaces sycl_be::attention_rows_quantized + attention_combine
 * (sycl_kernels.h:238-240) for the I8 format; key bias, groups, blocks, relative bias and anchored windows are not
 * taken. */
int xs_hip_attention_i8(void* stream, const float* q, const void* k_codes, const void* k_scales, const void* v_codes,
                        const void* v_scales, float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                        int64_t head_dim, int64_t kv_len, float scale, float softcap, int64_t window, int causal,
                        int64_t split, void* scratch);
/* No counterpart in the reference: for callers that capture a step into a HIP graph and replay it while the cache
 * grows. xs_hip_attention_i8 over a cache of kv_capacity keys of which kv_len[0] -- a device int64 read when the kernel
 * runs, clamped to [0, kv_capacity] -- are held; the caller keeps kv_len[0] >= tokens. `split` is fixed at the launch
 * (take xs_hip_attention_i8_split of the largest key count the replays will see); splits left without keys add
 * nothing. */
int xs_hip_attention_i8_at(void* stream, const float* q, const void* k_codes, const void* k_scales,
                           const void* v_codes, const void* v_scales, float* out, int64_t tokens, int64_t q_heads,
                           int64_t kv_heads, int64_t head_dim, int64_t kv_capacity, const int64_t* kv_len,
                           float scale, float softcap, int64_t window, int causal, int64_t split, void* scratch);
int64_t xs_hip_attention_i8_split(int64_t tokens, int64_t kv_heads, int64_t kv_len);
/* The split xs_hip_attention and xs_hip_attention_quantized (for pairs other than int8/int8) run best at for this shape:
 * about two workgroups a CU, each at least 128 keys. Scratch: xs_hip_attention_i8_scratch. */
int64_t xs_hip_attention_rows_split(int64_t tokens, int64_t kv_heads, int64_t kv_len);
/* No counterpart in the reference (its dispatch picks no split by format): the split at which the rows kernel for this
 * key format runs best -- three workgroups a CU for f16 keys (k_format XS_KV_FLOAT, kv_dtype XS_F16) and int8 keys at
 * head_dim <= 128 with at most 4 query heads a KV head, whose kernels are built for three; two, as
 * xs_hip_attention_rows_split, otherwise. For callers of
 * xs_hip_attention and xs_hip_attention_quantized that know the cache's format. */
int64_t xs_hip_attention_rows_split_kv(xs_kv_format k_format, xs_dtype kv_dtype, int64_t tokens, int64_t q_heads,
                                       int64_t kv_heads, int64_t kv_len, int64_t head_dim);
size_t xs_hip_attention_i8_scratch(int64_t tokens, int64_t q_heads, int64_t head_dim, int64_t split);
/* Decode attention over a float KV cache: keys and values [kv_len, kv_heads, head_dim] of kv_dtype (XS_F16 or XS_F32;
 * the Float KV format: f16 rows at f16 precision, f32 at f32), q and out as xs_hip_attention_i8, the same key
 * selection, scale, softcap, split and scratch (xs_hip_attention_i8_split, xs_hip_attention_i8_scratch) -- cpu_ref::
 * attention (ops.cpp:113-156, 535-594) over the rows the cache holds, f32 accumulation. Replaces
 * sycl_be::attention_rows<KV> with attention_combine (sycl_kernels.h, KV = half or float; dispatch
 * sycl_backend.cpp:2274-2290). q, out, k, v 16-byte aligned. */
int xs_hip_attention(void* stream, xs_dtype kv_dtype, const float* q, const void* k, const void* v, float* out,
                     int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_len, float scale,
                     float softcap, int64_t window, int causal, int64_t split, void* scratch);
/* xs_hip_attention over a cache of kv_capacity rows of which the kernel reads how many it holds from the device int64
 * at kv_len when it runs (clamped to [0, kv_capacity]): for steps replayed from captured HIP graphs. No reference
 * counterpart, as xs_hip_attention_i8_at. */
int xs_hip_attention_at(void* stream, xs_dtype kv_dtype, const float* q, const void* k, const void* v, float* out,
                        int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t kv_capacity,
                        const int64_t* kv_len, float scale, float softcap, int64_t window, int causal, int64_t split,
                        void* scratch);
/* Decode attention over a quantized cache of any pair of formats the reference reads (kv_formats_supported,
 * sycl_kernels.h:209-212): int8 keys and values (then exactly xs_hip_attention_i8), keys and values in the same
 * TurboQuant format, or int8 keys with TurboQuant values. Each stream as xs_hip_quantize_kv writes it: int8 codes
 * [kv_len, kv_heads, head_dim] with f32 scales [kv_len, kv_heads]; TurboQuant codes [kv_len * kv_heads *
 * head_dim / 128, 16 * bits] bytes with f16 norms [kv_len * kv_heads * head_dim / 128]. cpu_ref::attention over the
 * values the cache stores (quant::round_trip_kv, kv_format.cpp:57-61), computed in the formats' rotated domain: the
 * query rotated as the rows are, the weighted sum rotated back. q, out, key selection, scale, softcap, split and
 * scratch as xs_hip_attention_i8; with TurboQuant values head_dim is 128, 256 or 512. Codes 16-byte aligned. Other
 * pairs are refused with XS_HIP_EUNSUPPORTED ("keys in <k> with values in <v>"). Replaces
 * sycl_be::attention_rows_quantized + attention_combine (sycl_kernels.h:236-240; rows as sycl_kv_rows.h:37-100). */
int xs_hip_attention_quantized(void* stream, xs_kv_format k_format, xs_kv_format v_format, const float* q,
                               const void* k_codes, const void* k_scales, const void* v_codes, const void* v_scales,
                               float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                               int64_t kv_len, float scale, float softcap, int64_t window, int causal, int64_t split,
                               void* scratch);
/* xs_hip_attention_quantized over a cache of kv_capacity keys of which the kernel reads how many it holds from the
 * device int64 at kv_len (clamped to [0, kv_capacity]). No reference counterpart, as xs_hip_attention_i8_at. */
int xs_hip_attention_quantized_at(void* stream, xs_kv_format k_format, xs_kv_format v_format, const float* q,
                                  const void* k_codes, const void* k_scales, const void* v_codes,
                                  const void* v_scales, float* out, int64_t tokens, int64_t q_heads, int64_t kv_heads,
                                  int64_t head_dim, int64_t kv_capacity, const int64_t* kv_len, float scale,
                                  float softcap, int64_t window, int causal, int64_t split, void* scratch);
/* xs_hip_attention_i8 with no scratch argument and no allocation: a split's partial rows go to a device array of
 * 8 MiB (8388608 bytes) that the library holds on each GPU it runs on until the process ends; a split needing more
 * (xs_hip_attention_i8_scratch bytes) is refused with XS_HIP_EINVAL. No reference counterpart: it is for callers that
 * cannot allocate device memory -- code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. Same results as xs_hip_attention_i8 (the same kernels). Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, or two host threads) race. */
int xs_hip_attention_i8_noalloc(void* stream, const float* q, const void* k_codes, const void* k_scales,
                                const void* v_codes, const void* v_scales, float* out, int64_t tokens, int64_t q_heads,
                                int64_t kv_heads, int64_t head_dim, int64_t kv_len, float scale, float softcap,
                                int64_t window, int causal, int64_t split);

/* ---- Split-attention combine and merge (the reference's partial-row layout) ------------------------------------ */

/* part [rows, split, head_dim + 2]: per row and split, head_dim unnormalized weighted sums, the split's max and its sum
 * of exponentials relative to it (max -inf: a split that saw no key). out [rows, head_dim] = the splits merged and
 * normalized. Replaces sycl_be::attention_combine (sycl_kernels.h:240; sycl_kernels.cpp:1975-1995). */
int xs_hip_attention_combine(void* stream, const float* part, float* out, int64_t rows, int64_t split,
                             int64_t head_dim);
/* acc [rows, head_dim + 2], a partial row in the same layout, takes in each row's `split` partial rows of `part`;
 * first != 0 starts acc as their merge alone. xs_hip_attention_combine(acc, split 1) then gives the output. Replaces
 * sycl_be::attention_merge (sycl_kernels.h:241-244; sycl_kernels.cpp:1997-2030). */
int xs_hip_attention_merge(void* stream, const float* part, float* acc, int64_t rows, int64_t split, int64_t head_dim,
                           int first);

/* ---- Data movement: gather, transpose, concat ------------------------------------------------------------------ */

/* out [n, width] = rows ids[r] of table [rows, width] -- an embedding lookup. table f32, f16 or bf16 gives f32 rows
 * (f16 / bf16 widened exactly); an i32 table gives its rows' bits as they are (i32 out). ids i32 or i64. An id outside
 * [0, rows) gives a row of zeros (cpu-ref refuses it by name; the device keeps every access inside the table).
 * cpu_ref::gather (ops.cpp:157-173, cpu_backend.cpp:370); replaces sycl_be::gather / gather_bits
 * (sycl_kernels.h:106-110). */
int xs_hip_gather(void* stream, xs_dtype table_dtype, const void* table, int64_t rows, int64_t width,
                  xs_dtype ids_dtype, const void* ids, int64_t n, void* out);
/* y = x with its axes permuted: y.shape[i] = in_shape[perm[i]], elements of elem_bytes (1, 2, 4 or 8) moved as they
 * are; rank 1 to XS_MAX_RANK. cpu_ref::transpose (ops.cpp:312-340); replaces sycl_be::transpose (sycl_kernels.h:
 * 121-128). */
int xs_hip_transpose(void* stream, const void* x, void* y, int64_t elem_bytes, int rank, const int64_t* in_shape,
                     const int32_t* perm);
/* The parts joined along an axis: `outer` rows (the product of the dims before the axis), each the parts' rows laid
 * end to end -- part k contributes part_row_bytes[k] bytes from parts[k] + o * part_row_bytes[k]. 1 to
 * XS_CONCAT_PARTS parts, any element type. cpu_ref::concat (ops.cpp:616-637); replaces sycl_be::concat
 * (sycl_kernels.h:95-104, kConcatParts). */
#define XS_CONCAT_PARTS 8
int xs_hip_concat(void* stream, int count, const void* const* parts, const int64_t* part_row_bytes, void* out,
                  int64_t outer);

/* ---- Strided copy -------------------------------------------------------------------------------------------- */

/* y[r, :] = x[r, :] for `rows` rows of `row_bytes` bytes, x rows `x_row_stride` bytes apart and y rows `y_row_stride`
 * apart: a graph Slice on an inner axis, materialized. Replaces sycl_be::slice (sycl_kernels.h:119-120): its
 * (outer, dim, begin, len, inner) are rows = outer, x + begin * inner * elem, x_row_stride = dim * inner * elem,
 * row_bytes = len * inner * elem. */
int xs_hip_copy_rows(void* stream, const void* x, int64_t x_row_stride, void* y, int64_t y_row_stride, int64_t rows,
                     int64_t row_bytes);

/* ---- Measurement helper -------------------------------------------------------------------------------------- */

/* y = x, `bytes` bytes (a multiple of 16, 16-byte aligned), with the 128-bit streaming loads and stores of the
 * kernels above: the known-size kernel hardware byte counters are calibrated against. No reference counterpart. */
int xs_hip_copy(void* stream, const void* x, void* y, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* XS_HIP_H */
