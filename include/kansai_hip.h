/*
 * kansai_hip.h -- C ABI of the MI355X (gfx950) HIP backend for Kansai's
 * int8 quantize -> int8 matmul -> dequantize path and its fp32 matmul.
 *
 * Contract (mirrors the reference's backend contract,
 * backend/metal/include/kansai/backend/metal/MetalOps.hpp:13-88):
 *   - plain pointers and int64 sizes; no C++ or torch types;
 *   - tensor pointers are DEVICE pointers (from kh_alloc, or any device
 *     allocation on the current device) unless named host_*; outputs are
 *     caller-allocated; the library never frees caller memory;
 *   - every function returns an int status, KH_OK (0) on success; on
 *     failure kh_last_error() gives a message (thread-local);
 *   - compute calls are ordered on the library stream of the current
 *     device; kh_synchronize() waits for them and reports data errors
 *     found on the device (a non-finite value given to a quantizer), the
 *     asynchronous counterpart of the reference raising ValueError from
 *     round(nan) (python/kansai/quantize.py:69).
 *   - row-major, contiguous tensors, as the reference's Tensor
 *     (core/include/kansai/Tensor.hpp:228-237).
 *
 * Quantization arithmetic is the reference's exactly
 * (python/kansai/quantize.py:66-70, :76):
 *   m = max|v|; scale = m / 127.0 (binary64) if m > 0 else 1.0;
 *   q = clamp(round_half_even((double)v / scale), -127, 127);
 *   dequantized = (float)((double)q * scale).
 * Scales are binary64 device arrays, like the reference's Python float.
 */
#ifndef KANSAI_HIP_H
#define KANSAI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KH_OK 0
#define KH_ERR_NO_DEVICE 1     /* no gfx950 device / library not initialised */
#define KH_ERR_INVALID_ARG 2   /* shape, pointer or alignment problem */
#define KH_ERR_OOM 3           /* device allocation failed */
#define KH_ERR_NONFINITE 4     /* NaN/inf reached a quantizer */
#define KH_ERR_HIP 5           /* any other HIP runtime error */

/* ---- device, errors --------------------------------------------------- */

/* kan::metal::available() (MetalOps.hpp:15-18): 1 if a gfx950 device is
 * usable, else 0.  Never fails, never throws. */
int kh_available(void);

/* Binds the calling thread to `device` and creates its library stream and
 * scratch state.  Called implicitly by every entry point on device 0 if
 * never called. */
int kh_init(int device);

/* Last error message of the calling thread ("" if none). Replaces the
 * std::runtime_error text the reference throws (MetalOps.mm:259-261). */
const char* kh_last_error(void);

/* Device facts used for roofline denominators: name (gcnArchName),
 * compute units, peak engine clock (kHz), memory clock (kHz), bus width
 * (bits), total global memory (bytes). */
int kh_device_info(char* name, size_t name_len, int* cus, int* clock_khz,
                   int* mem_clock_khz, int* bus_width, size_t* total_mem);

/* Waits for all work queued on the library stream, then reports (and
 * clears) deferred device errors: returns KH_ERR_NONFINITE if a quantizer
 * met a NaN/inf since the previous synchronize. */
int kh_synchronize(void);

/* The library stream (a hipStream_t) of the current device, for callers
 * that record their own events or order their own work after it. */
int kh_get_stream(void** stream);

/* ---- device memory (hipMalloc-backed pool) ---------------------------- */

/* Device buffers from a caching pool: freed blocks are kept per size class
 * and reused, so a graph executed repeatedly stops calling hipMalloc after
 * its first run.  Replaces core/src/Storage.cpp:22-32 (page-aligned host
 * allocation) and the first-fit core/src/StoragePool.cpp:5-24 for device
 * memory.  Blocks are 256-byte aligned.  kh_free returns a block to the
 * pool (stream-ordered: it is reused only by later work on the same
 * stream).  kh_pool_trim gives all cached blocks back to the driver. */
int kh_alloc(size_t bytes, void** dptr);
int kh_free(void* dptr);
int kh_pool_trim(void);
/* bytes currently handed out, bytes cached in free lists, number of
 * hipMalloc calls made so far. */
int kh_pool_stats(size_t* in_use, size_t* cached, size_t* driver_allocs);
/* The number of kh_alloc calls served so far (from the free lists or the
 * driver), including the library's own (e.g. kh_gemm_i8's split-K partials).
 * No reference counterpart: it lets a caller check that a call drew nothing
 * from the pool (kh_linear_i8_noalloc). */
int kh_pool_requests(size_t* requests);
/* The library's own scratch area (absmax partials and the like, outside the
 * pool): its size in bytes, the number of requests made of it so far and
 * the number of hipMalloc calls it made.  No reference counterpart: the
 * reference has no device scratch; it lets a caller check that a call used
 * none (kh_linear_i8_noalloc). */
int kh_scratch_stats(size_t* bytes, size_t* requests, size_t* driver_allocs);

/* Copies.  kh_memcpy_h2d / kh_memcpy_d2h are synchronous with respect to
 * the host (they order after queued work on the library stream), as the
 * reference's synchronous backend calls are (MetalOps.mm:317).
 * kh_memcpy_d2d is stream-ordered. */
int kh_memcpy_h2d(void* dst, const void* host_src, size_t bytes);
int kh_memcpy_d2h(void* host_dst, const void* src, size_t bytes);
int kh_memcpy_d2d(void* dst, const void* src, size_t bytes);

/* ---- timing (HIP events on the library stream) ------------------------ */
int kh_event_create(void** event);
int kh_event_record(void* event);
int kh_event_elapsed_ms(void* start, void* end, float* ms);
int kh_event_destroy(void* event);

/* ---- graphs (HIP graph capture of the library stream) ------------------- */

/* Records the library calls made between kh_graph_capture_begin and
 * kh_graph_capture_end into a HIP graph instead of running them, and
 * instantiates it; kh_graph_launch replays the recorded kernels and copies
 * on the library stream with one host call.  Stands where the reference
 * re-interprets a cached traced graph on every call (python/kansai/kir.py:
 * 536-555 jit cache, 957-1068 run_planned): the planned run is recorded once
 * and replayed.  The graph reads and writes the very buffers the captured
 * calls named, so inputs are refreshed in place before a launch, and outputs
 * are overwritten by the next launch.  Pool blocks freed during the capture
 * belong to the graph (they return to the pool at kh_graph_destroy), and a
 * block still held at capture end stays the graph's when it is freed later,
 * so no other work is handed memory a launch writes.  Work needing a larger
 * scratch area or a host synchronisation cannot be captured (run it once
 * first); kh_synchronize, the host copies and kh_pool_trim fail while a
 * capture is open.  kh_graph_capture_end(NULL) discards the capture.
 * kh_graph_destroy waits for the stream first. */
int kh_graph_capture_begin(void);
int kh_graph_capture_end(void** graph);
int kh_graph_launch(void* graph);
int kh_graph_destroy(void* graph);

/* ---- quantize / dequantize -------------------------------------------- */

/* quantize_symmetric (python/kansai/quantize.py:50-70) over a whole
 * tensor of n fp32 values: one scale, written to scale[0].  Up to 64 K
 * elements (x 16-byte and q 4-byte aligned) in one launch, larger tensors in
 * two passes (absmax partials, then the codes). */
int kh_quantize_tensor(const float* x, int64_t n, int8_t* q, double* scale);

/* The two passes of kh_quantize_tensor taken apart, so the absmax pass can
 * ride along with the kernel that produced x (the *_ex entry points below):
 * kh_absmax_parts writes up to max_parts partial maxima of |x| (as IEEE bit
 * patterns; NaN/inf sort above every finite value) and their count;
 * kh_quantize_tensor_parts reduces `nparts` of them to the tensor's absmax
 * and quantizes exactly as kh_quantize_tensor does.  Internal to the fused
 * graph path; no reference counterpart (the reference's quantize_symmetric
 * is one Python function, quantize.py:50-70). */
int kh_absmax_parts(const float* x, int64_t n, unsigned* parts, int max_parts, int* nparts);
int kh_quantize_tensor_parts(const float* x, int64_t n, const unsigned* parts, int nparts, int8_t* q,
                             double* scale);

/* quantize_symmetric applied to each row of a [rows, cols] matrix: one
 * scale per row (per token).  scales has `rows` entries. */
int kh_quantize_rows(const float* x, int64_t rows, int64_t cols, int8_t* q, double* scales);

/* quantize_symmetric applied to each column of an nn.Linear weight
 * (python/kansai/nn.py:74-81 lays it out [in = k, out = n], so a column
 * is one output channel).  Codes are written packed K-contiguous for the
 * GEMM: q_packed[j * k + i] = code of w[i, j]; scales has n entries. */
int kh_quantize_cols_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scales);

/* Per-tensor scale (one scale for the whole weight, as the reference's
 * QTensor.from_tensor, quantize.py:95-98) with the same K-contiguous
 * packing as kh_quantize_cols_packed. */
int kh_quantize_tensor_packed(const float* w, int64_t k, int64_t n, int8_t* q_packed, double* scale);

/* dequantize (quantize.py:73-77): out[i] = (float)((double)q[i] * scale[0]). */
int kh_dequantize_tensor(const int8_t* q, int64_t n, const double* scale, float* out);

/* Per-row dequantize: out[r, c] = (float)((double)q[r, c] * scales[r]). */
int kh_dequantize_rows(const int8_t* q, int64_t rows, int64_t cols, const double* scales, float* out);

/* Dequantize of a packed per-column weight back to the [k, n] fp32 layout
 * the reference's qlinear multiplies with (quantize.py:115-122):
 * out[i, j] = (float)((double)q_packed[j * k + i] * scales[scales_n == 1 ? 0 : j]). */
int kh_dequantize_packed(const int8_t* q_packed, int64_t k, int64_t n, const double* scales,
                         int64_t scales_n, float* out);

/* ---- int8 GEMM with fused dequantize + bias epilogue ------------------- */

/* acc[i, j] = sum_k a[i, k] * b_packed[j, k]   (int32, exact)
 * out[i, j] = (float)((double)acc[i, j] * (sa_i * sb_j)) + bias[j]
 * a: [M, K] int8 row-major (quantized activations); b_packed: [N, K] int8
 * (a packed weight from kh_quantize_*_packed).  sa has M entries when
 * sa_per_row != 0 else 1; sb has N entries when sb_per_col != 0 else 1
 * (binary64, device).  bias (fp32 [N], device) may be NULL.  out (fp32
 * [M, N]) may be NULL; acc_out (int32 [M, N]) may be NULL; at least one of
 * them must be given.  The reference has no int8 GEMM (quantize.py:30-44):
 * this replaces its x.matmul(dequantize(W)).add(bias)
 * (quantize.py:115-122) on the int8 path.  K <= 133144 keeps the int32
 * accumulator exact.  Skinny shapes (M <= 64) whose 16-column tiles leave
 * CUs idle (N < 16 x CUs / 2) with K >= 8192 split K across workgroups:
 * int32 partials in pooled device memory, summed (exactly) by a second
 * launch that applies the epilogue. */
int kh_gemm_i8(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K,
               const double* sa, int sa_per_row, const double* sb, int sb_per_col,
               const float* bias, float* out, int32_t* acc_out);

/* kh_gemm_i8's output with the graph's next elementwise steps fused into
 * the epilogue, in the order the reference applies them:
 *   y = (float)((double)acc * (sa_i * sb_j)) + bias[j];
 *   y = act(y)            act: KH_ACT_NONE or KH_ACT_GELU (the erf form of
 *                         backend/cpu/src/Ops.cpp:250-256, to ~1e-7 * max(1, |x|));
 *   out = residual + y    when residual (fp32 [M, N]) is not NULL -- the
 *                         pre-LN block's x.add(linear(..)), nn.py:466-478.
 * absmax_parts (may be NULL): up to max_parts partial maxima of |out| for
 * kh_quantize_tensor_parts, count in *nparts. */
#define KH_ACT_NONE 0
#define KH_ACT_GELU 1
int kh_gemm_i8_ex(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K,
                  const double* sa, int sa_per_row, const double* sb, int sb_per_col,
                  const float* bias, int act, const float* residual, float* out,
                  unsigned* absmax_parts, int max_parts, int* nparts);

/* kh_gemm_i8_ex's fp32 result quantized per tensor, as kh_quantize_tensor
 * would quantize it (quantize.py:50-70 on the output of qlinear and the
 * pre-LN block's GELU / residual, nn.py:466-478), without the fp32 result
 * ever being written: codes int8 [M, N] into q, the binary64 scale into
 * *scale.  Two passes over the GEMM (absmax, then quantize), which is the
 * cheaper order when the fp32 output would be read again only to be
 * quantized (the graph's fc1 -> GELU -> quantize).  Uses the library's
 * scratch area; a NaN/inf result reports KH_ERR_NONFINITE at the next
 * synchronize, as kh_quantize_tensor does. */
int kh_gemm_i8_quant(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K,
                     const double* sa, int sa_per_row, const double* sb, int sb_per_col,
                     const float* bias, int act, const float* residual, int8_t* q, double* scale);

/* kh_gemm_i8_ex's fp32 result quantized per row (per token), as
 * kh_quantize_rows would quantize it (quantize.py:50-70 applied to each row
 * of qlinear's output, quantize.py:115-122, and its GELU, nn.py:466-478),
 * without the fp32 result ever being written: codes int8 [M, N] into q, the
 * M binary64 row scales into scales.  A workgroup owns 32 whole rows and
 * keeps their results in registers between the row absmax and the codes; it
 * takes N = 512, 1024 or 1536 and K = 256 or 384 (the per-token fc1 of a
 * small model, 16-byte aligned operands); other shapes run
 * kh_gemm_i8_ex into a pooled temporary and kh_quantize_rows.  A NaN/inf row
 * reports KH_ERR_NONFINITE at the next synchronize.  No reference
 * counterpart (the reference has no per-token quantize). */
int kh_gemm_i8_quant_rows(const int8_t* a, const int8_t* b_packed, int64_t M, int64_t N, int64_t K,
                          const double* sa, int sa_per_row, const double* sb, int sb_per_col,
                          const float* bias, int act, int8_t* q, double* scales);

/* The per-tensor quantize of an fp32 activation fused into the GEMM that
 * consumes it:kh_quantize_tensor_parts(x, x_parts) (quantize.py:50-70 on
 * the activation, with the absmax partials its producer wrote) followed by
 * kh_gemm_i8_ex(codes, b_packed, sa = that scale, ...) (qlinear's int8
 * matmul and dequantize, quantize.py:115-144, with the fused bias / GELU /
 * residual), without the codes ever being written.  x fp32 [M, K] (16-byte
 * aligned for the fused kernel); x_parts: the producer's partials (at least
 * one); x_scale (may be NULL) receives the activation's binary64 scale;
 * absmax_parts as kh_gemm_i8_ex.  The same outputs as the two calls (other
 * shapes run them).  A NaN/inf in x reports KH_ERR_NONFINITE at the next
 * synchronize, as kh_quantize_tensor_parts does. */
int kh_gemm_i8_qload(const float* x, int64_t M, int64_t N, int64_t K, const unsigned* x_parts, int x_nparts,
                     const int8_t* b_packed, const double* sb, int sb_per_col, const float* bias, int act,
                     const float* residual, float* out, double* x_scale, unsigned* absmax_parts, int max_parts,
                     int* nparts);

/* kh_gemm_i8_qload with one scale per row of x (per token): row i is
 * quantized with the scale of its own absmax (quantize.py:50-70 applied to
 * the row), taken from the producer's partials row_parts [M, parts_per_row]
 * (the max |x| bits of pieces of each row, e.g. kh_attention_rows' one word
 * per head), inside the GEMM that consumes x, so the codes are never
 * written; the epilogue then uses sa_i * sb_j.  x_scales (may be NULL)
 * receives the M binary64 row scales.  The same outputs as
 * kh_quantize_rows followed by kh_gemm_i8_ex with per-row scales (which run
 * for shapes the fused kernel does not take: M a multiple of 64, N = 128,
 * 256 or a multiple of 384, K of 64, parts_per_row <= 16).  A NaN/inf row
 * reports KH_ERR_NONFINITE at the next synchronize.  No reference
 * counterpart (the reference has no per-token quantize). */
int kh_gemm_i8_qload_rows(const float* x, int64_t M, int64_t N, int64_t K, const unsigned* row_parts,
                          int parts_per_row, const int8_t* b_packed, const double* sb, int sb_per_col,
                          const float* bias, int act, const float* residual, float* out, double* x_scales);

/* Per-token activation quantize fused into the GEMM's producer: x fp32
 * [M, K] is quantized per row into q_scratch (int8 [M, K]) and
 * sx_scratch (binary64 [M]), then kh_gemm_i8 runs with sa = sx_scratch
 * (per row).  The decode-style entry point of config C5.  One launch for
 * M <= 3 (M <= 2 with K = 2048, 4096 or 8192; M = 3 with K = 2048 or
 * 4096, 16-byte aligned x and b_packed), two otherwise. */
int kh_linear_i8(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N,
                 const double* sb, int sb_per_col, const float* bias,
                 int8_t* q_scratch, double* sx_scratch, float* out);

/* The int8 Linear with a per-tensor activation scale (config C1's QLinear
 * with act_granularity "tensor"): x fp32 [M, K] quantized with one scale
 * over the whole tensor (quantize.py:50-70) into q_scratch (int8 [M, K]) and
 * sx_scratch[0] (binary64), then kh_gemm_i8 with sa = that scale, per-tensor
 * (qlinear, quantize.py:115-122, with the dequantize and bias fused).  One
 * launch for M <= 64, K = 512, 1024, 2048 or 4096 and M * K <= 32768
 * (every workgroup quantizes the whole of x itself); kh_quantize_tensor then
 * kh_gemm_i8 otherwise.  A NaN/inf in x reports KH_ERR_NONFINITE at the next
 * synchronize. */
int kh_linear_i8_tensor(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N,
                        const double* sb, int sb_per_col, const float* bias,
                        int8_t* q_scratch, double* sx_scratch, float* out);

/* kh_linear_i8 for callers that cannot allocate device memory (code under
 * HIP graph capture, tight decode loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference.  The per-row codes and scales go to a
 * fixed array compiled into the library (2 MiB of codes + 2048 binary64
 * scales, one copy per device for the life of the process) instead of
 * q_scratch / sx_scratch: calls with M > 2048 or M * K > 2 MiB are
 * rejected (KH_ERR_INVALID_ARG).  Allocates nothing and never initialises
 * a device: call kh_init (or any other entry point) on the device first,
 * else KH_ERR_NO_DEVICE.  Output is identical to kh_linear_i8's.  Every
 * call on a device shares its one array, which keeps the last call's
 * codes; calls are ordered on the library stream, so calls that overlap
 * on one GPU (a graph holding this call replayed outside the library
 * stream, say) race on it. */
int kh_linear_i8_noalloc(const float* x, int64_t M, int64_t K, const int8_t* b_packed, int64_t N,
                         const double* sb, int sb_per_col, const float* bias, float* out);

/* The epilogue alone, for an int8_matmul whose dequantize was not fused:
 * out[i, j] = (float)((double)acc[i, j] * (sa_i * sb_j)) [+ bias[j]].
 * quantize.py:76 applied to an accumulator. */
int kh_dequantize_acc(const int32_t* acc, int64_t M, int64_t N, const double* sa, int sa_per_row,
                      const double* sb, int sb_per_col, const float* bias, float* out);

/* ---- fp32 matmul ------------------------------------------------------- */

/* out (M, N) = a (M, K) @ b (K, N) [+ bias (N)], fp32 row-major; the
 * signature of kan::metal::matmul / matmul_mps (MetalOps.hpp:27, 35) and
 * kan::cpu::matmul (backend/cpu/src/Ops.cpp:322-339), with the bias add
 * of Ops.cpp:34-38 fused when bias != NULL. */
int kh_matmul_f32(const float* a, const float* b, float* out, int64_t M, int64_t K, int64_t N,
                  const float* bias);

/* ---- fp32 elementwise around the path ----------------------------------- */

/* out[i] = a[i] + b[i]: kan::metal::add (MetalOps.hpp:51),
 * kan::cpu::add (backend/cpu/src/Ops.cpp:22-24). */
int kh_add(const float* a, const float* b, float* out, int64_t n);

/* out[i, j] = x[i, j] + bias[j], then (v > 0 ? v : 0) when relu != 0:
 * kan::metal::add_bias / bias_relu (MetalOps.hpp:37-43),
 * kan::cpu::add_bias_broadcast (Ops.cpp:34-38), fused_bias_relu
 * (backend/cpu/src/Fused.cpp:5-14). */
int kh_add_bias(const float* x, const float* bias, float* out, int64_t batch, int64_t features, int relu);

/* out[i] = x[i] > 0 ? x[i] : 0: kan::metal::relu (MetalOps.hpp:54),
 * kan::cpu::relu_fwd (backend/cpu/src/Ops.cpp:197-199). */
int kh_relu(const float* x, float* out, int64_t n);

/* ---- fp32 pieces of a decoder block (config C4) -------------------------- */

/* out[r, :] = tok[ids[r], :] + pos[r % T, :] -- nn.Embedding lookups summed
 * (python/kansai/nn.py:624-646; examples/tinyshakespeare/
 * train_shakespeare_large.py:72-75).  ids: int32 [rows]; tok [V, D];
 * pos [T, D].  An id outside [0, V) is reported by kh_synchronize
 * (KH_ERR_INVALID_ARG). */
int kh_embedding(const int32_t* ids, int64_t rows, int T, const float* tok, int V, const float* pos, int D,
                 float* out);

/* LayerNorm over the last axis (nn.py:308-331): biased variance,
 * (x - mean) / sqrt(var + eps) * weight + bias.  D <= 1024. */
int kh_layernorm(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps, float* out);
/* ... also writing absmax partials of out (see kh_absmax_parts). */
int kh_layernorm_ex(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps,
                    float* out, unsigned* absmax_parts, int max_parts, int* nparts);
/* LayerNorm followed by the per-tensor quantize of its output
 * (quantize.py:50-70 on nn.LayerNorm's result, the pre-LN block's
 * x -> ln -> Linear input, nn.py:466-478), without writing the fp32
 * output: two passes over x (absmax, then quantize), codes int8
 * [rows, D] into q and the binary64 scale into *scale.  Codes equal
 * kh_quantize_tensor of kh_layernorm's output bit for bit. */
int kh_layernorm_quant(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps,
                       int8_t* q, double* scale);
/* LayerNorm (as kh_layernorm) with its output quantized per row -- per token
 * -- in one pass: scales[r] = max_j |y[r,j]| / 127 in binary64 (1.0 for an
 * all-zero row) and q[r,j] = clamp(round_half_even(y[r,j] / scales[r]),
 * -127, 127), quantize_symmetric (quantize.py:50-70) applied to each row of
 * nn.LayerNorm's output (nn.py:308-331).  The fp32 values are never stored.
 * No reference counterpart as one call: the reference quantizes activations
 * per tensor only; this is the per-token producer fusion for callers that
 * choose per-row activation scales. */
int kh_layernorm_quant_rows(const float* x, int64_t rows, int D, const float* weight, const float* bias, float eps,
                            int8_t* q, double* scales);

/* Exact-erf GELU (backend/cpu/src/Ops.cpp:250-256). */
int kh_gelu(const float* x, float* out, int64_t n);

/* Causal multi-head self-attention core of nn.MultiHeadAttention.forward
 * (nn.py:381-427) with the additive causal mask of
 * train_shakespeare_large.py:69-70: per head softmax(Q K^T / sqrt(dk) +
 * mask) V.  qkv: [B*T, 3*H*dk], the fused Q|K|V projection (head h of Q at
 * columns h*dk..); out: [B*T, H*dk] with heads merged in place.  dk == 64. */
int kh_causal_attention(const float* qkv, int B, int T, int H, int dk, float* out);
/* ... also writing absmax partials of out (see kh_absmax_parts). */
int kh_causal_attention_ex(const float* qkv, int B, int T, int H, int dk, float* out, unsigned* absmax_parts,
                           int max_parts, int* nparts);
/* The same with the mask chosen by the caller: causal = 1 as above, causal = 0
 * attends over all T keys -- BigGPT.forward passes no mask when the sequence
 * is shorter than its position table (train_shakespeare_large.py:86). */
int kh_attention_ex(const float* qkv, int B, int T, int H, int dk, int causal, float* out, unsigned* absmax_parts,
                    int max_parts, int* nparts);
/* kh_attention_ex(causal) writing, instead of per-tensor partials, the max
 * |out| bits of every (row, head): row_parts [B*T, H] -- what a following
 * per-row (per-token) quantize of out needs (the row's absmax is the max of
 * its H words; kh_gemm_i8_qload_rows reads them). */
int kh_attention_rows(const float* qkv, int B, int T, int H, int dk, int causal, float* out, unsigned* row_parts);
/* Attention with the caller's additive mask, the reference's contract
 * (nn.py:421-422: scores = q k^T / sqrt(dk) + mask, then softmax), with or
 * without the causal mask on top.  mask: fp32, element (b, h, i, j) at
 * b*stride_b + h*stride_h + i*stride_q + j (a stride 0 broadcasts that axis,
 * e.g. the reference's [1, 1, T, T] causal mask: 0, 0, T; keys contiguous),
 * mask_elems elements in all.  -inf entries give probability 0; a row masked
 * everywhere gives NaN, as the reference's softmax does.  row_parts (may be
 * NULL): kh_attention_rows' per-(row, head) partials. */
int kh_attention_masked(const float* qkv, int B, int T, int H, int dk, int causal, const float* mask,
                        int64_t mask_elems, int64_t stride_b, int64_t stride_h, int64_t stride_q, float* out,
                        unsigned* row_parts);

/* ---- measurement utility (no reference counterpart) ------------------- */

/* The int8 MFMA rate this device sustains on the given operand bytes and the
 * shader clock it runs at meanwhile: one workgroup per CU, 8 waves, each
 * issuing `iters` x 16 independent v_mfma_i32_32x32x32_i8 on 8 operand
 * registers loaded once from `operands` (16-byte aligned, at least
 * compute-units x 64 KiB).  Synchronous.  Used by bench.py to state the
 * attainable int8 peak next to the published one. */
int kh_probe_mfma_i8(const int8_t* operands, int64_t bytes, int64_t iters, double* tops, double* clock_mhz);

/* Reads `bytes` (16-byte aligned, a multiple of 16, below 2 GiB) as the
 * weight-streaming GEMMs read their weights -- every workgroup issues all of
 * its 64 KiB of loads up front -- and discards them.  Asynchronous on the
 * library stream, so it can be timed back to back like kh_linear_i8: the
 * practical ceiling bench.py states for the decode rows. */
int kh_probe_stream_read(const void* p, int64_t bytes);

#ifdef __cplusplus
}
#endif
#endif /* KANSAI_HIP_H */
