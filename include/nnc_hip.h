/* nnc_hip.h — the C ABI of libnnc_hip.so: nnc's attention op on one AMD
 * Instinct MI355X (gfx950) GPU.
 *
 * nnc has no op registry: its attention "op" is the trio
 * nnc_attn_block / nnc_attn_merge / nnc_attn_finish (reference
 * src/libnnc/nn_ops.h:31-61) driven by the attention core of
 * attention_forward (reference src/libnnc/model.cpp:1693-1761) over the
 * per-layer K/V buffers that model_kv_init sizes (reference
 * src/libnnc/model.h:226-326, model.cpp:1891-2041). A per-block call is too
 * fine-grained for a GPU, so this library replaces that core at layer
 * granularity: one call per (layer, forward pass) computes, for every query
 * token t of the batch and every query head h,
 *
 *   out[t][h] = sum over k in span(pos0 + t) of softmax_k(scale * q[t][h] . K[k]) * V[k]
 *
 * with the span of model_attn_span (reference model.cpp:2300-2316), KV head
 * h / (n_head / n_kv), and key k stored in row k % rows of the layer's
 * buffer. The K/V layout and element types are nnc's own, unchanged:
 * token-major rows of kv_dim = n_kv * head_dim elements, BF16 (uint16 bit
 * patterns, round-to-nearest-even from F32) or F32 (reference nnc.h:199-203,
 * runtime.h:97-113).
 *
 * Errors follow nnc's convention (reference nnc.cpp:24-43, runtime.h:29-46):
 * every call returns an nnc_status, a failure records a message readable with
 * nnc_hip_last_error() on the calling thread, and nothing throws across the
 * ABI. The status values are nnc.h's own; no new status is added.
 *
 * Threading: one nnc_hip_kv belongs to one session, which one thread drives
 * at a time (reference nnc.h:27-32). Each cache owns one HIP stream; calls on
 * one cache are ordered on it. Separate caches may be used from separate
 * threads at once.
 */
#ifndef NNC_HIP_H
#define NNC_HIP_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef NNC_H
/* The status codes of reference nnc.h:50-61, same names and values. When
 * nnc.h is included first, its own definition is used. */
typedef enum nnc_status
{
	NNC_OK = 0,
	NNC_ERR_INVALID_ARGUMENT = 1,
	NNC_ERR_UNSUPPORTED_CPU = 2,
	NNC_ERR_IO = 3,
	NNC_ERR_BAD_FORMAT = 4,
	NNC_ERR_UNSUPPORTED_MODEL = 5,
	NNC_ERR_OUT_OF_MEMORY = 6,
	NNC_ERR_CONTEXT_FULL = 7,
	NNC_ERR_CANCELLED = 8,
} nnc_status;
#endif

/* Log levels, the values of nnc_log_level (reference nnc.h:83-89). */
#define NNC_HIP_LOG_DEBUG 0
#define NNC_HIP_LOG_INFO 1
#define NNC_HIP_LOG_WARN 2
#define NNC_HIP_LOG_ERROR 3

/* Receives one complete message without a trailing newline; the signature
 * of nnc_log_callback (reference nnc.h:91-92), so nnc's own callback can be
 * passed straight through. */
typedef void (*nnc_hip_log_callback)(int level, const char* message, void* user);

/* Routes the bridge's diagnostics to `callback`; NULL restores the default,
 * which writes warnings and errors to stderr (reference nnc.h:94-98,
 * nnc_set_log_callback). Failures are still reported through return values
 * and nnc_hip_last_error(). nnc_hip_kv_create logs, at INFO, the device and
 * the device memory the cache holds (the counterpart of nnc's context line,
 * reference session.cpp:341-343). */
void nnc_hip_set_log_callback(nnc_hip_log_callback callback, void* user);

/* A session's K/V cache in device memory: one buffer per cache-owning layer,
 * as in model_kv_cache::bufs (reference model.h:252-326). */
typedef struct nnc_hip_kv nnc_hip_kv;

/* Allocates n_buf K/V buffers in HBM, buffer i holding rows[i] rows of
 * kv_dim[i] elements (BF16 when bf16, else F32), zero-filled, plus one HIP
 * stream. Mirrors model_kv_init's buffer allocation (reference
 * model.cpp:1908-1957; rows come from the same rule: n_ctx, or a ring of
 * round_up(window + n_batch, 256) rows for a sliding layer). A BF16 cache
 * also keeps an fp16 copy of every V buffer, written by every append, for the
 * prefill kernel, which uses it while every value in it is within +-8, where
 * P rounded to fp16 moves an output by at most 2^-11 * 8 = 3.9e-3 (1.5
 * times the device memory of K and V alone; NNC_HIP_F16_SHADOW=0 in the
 * environment at creation leaves it out, and prefill then runs slower). The
 * nnc-visible buffers stay BF16 in nnc's layout.
 * NNC_ERR_INVALID_ARGUMENT: n_buf <= 0, a NULL pointer, rows or kv_dim <= 0.
 * NNC_ERR_OUT_OF_MEMORY: the device allocation failed.
 * NNC_ERR_UNSUPPORTED_CPU: no usable HIP device (the nearest existing status:
 * this machine cannot run the op). */
nnc_status nnc_hip_kv_create(int32_t n_buf, const int32_t* rows, const int32_t* kv_dim, bool bf16,
                             nnc_hip_kv** out);

/* Frees the buffers, the scratch and the stream. NULL is a no-op. */
void nnc_hip_kv_free(nnc_hip_kv* kv);

/* Total device bytes held by the K/V buffers, fp16 copies included
 * (reference model.h:325, bytes). */
uint64_t nnc_hip_kv_bytes(const nnc_hip_kv* kv);

/* How the cache's attend calls compute batches of more than 16 tokens.
 * exact = false (the default): a BF16 batch runs the prefill kernel, within
 * the parity bound of nnc's CPU result but not bit-identical to the same
 * tokens' one-token calls. exact = true: every batch runs the split-K decode
 * kernels with each token on the split grid of its one-token call, so a
 * token's result has the same bits whatever batch computes it, the promise
 * nnc's CPU path keeps (reference model.cpp:1724-1729, docs/design.md:417-419)
 * for its n_batch-sized chunks and model_embed; prompt-sized batches then
 * cost several times more. Batches of up to 16 tokens (every batch of a
 * session, MTP verification included) take the exact path either way.
 * No counterpart in the reference, whose CPU path has only the exact mode;
 * for callers that need its bits on long batches.
 * NNC_ERR_INVALID_ARGUMENT: kv is NULL. */
nnc_status nnc_hip_kv_set_exact_batches(nnc_hip_kv* kv, bool exact);

/* Writes n_tok rows for positions pos0 .. pos0 + n_tok - 1 into buffer
 * `buf`, position p to row p % rows, from host memory already in the cache's
 * element type (the KV append of reference model.cpp:1662-1691, whose BF16
 * rounding is nnc_f32_to_bf16). k_rows and v_rows hold n_tok * kv_dim
 * elements each. Asynchronous on the cache's stream; the host rows may be
 * reused when the call returns (they are staged).
 * NNC_ERR_INVALID_ARGUMENT: bad buffer index, n_tok <= 0, pos0 < 0, NULL rows,
 * or n_tok > rows (the batch would overwrite itself). */
nnc_status nnc_hip_kv_append(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, const void* k_rows,
                             const void* v_rows);

/* As nnc_hip_kv_append, from F32 rows in host memory; a BF16 cache rounds
 * them on the device with round-to-nearest-even, giving the bits of
 * nnc_f32_to_bf16 (reference runtime.h:106-113). */
nnc_status nnc_hip_kv_append_f32(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, const float* k_rows,
                                 const float* v_rows);

/* As nnc_hip_kv_append_f32 with k_rows / v_rows in device memory. */
nnc_status nnc_hip_kv_append_f32_device(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok,
                                        const float* k_rows, const float* v_rows);

/* Parameters of the pre-attention step (nnc_hip_kv_prep_append_device): the
 * per-layer values attention_forward reads from the model (reference
 * model.cpp:1616-1660). The gammas are device memory; the frequency factors
 * are host memory (the rotation angles are formed on the host, see below). */
typedef struct nnc_hip_prep
{
	int32_t n_head; /* query heads */
	int32_t n_kv; /* KV heads; n_kv * head_dim is the buffer's kv_dim */
	int32_t head_dim; /* 1 .. 512 */
	const float* q_gamma; /* device: head_dim floats (attn_q_norm), or NULL: no Q norm */
	const float* k_gamma; /* device: head_dim floats (attn_k_norm), or NULL: no K norm */
	int32_t v_norm; /* nonzero: RMS-normalise V per head with no gamma (Gemma 4) */
	float rms_eps; /* hparams.rms_eps */
	int32_t n_rot; /* rotated values per head (L.n_rot): even, <= head_dim; 0: no RoPE */
	float freq_base; /* RoPE base (the layer's freq) */
	float pos_scale; /* RoPE position = (pos0 + t) * pos_scale (the layer's rope scale) */
	int32_t rope_mode; /* 0 NEOX, 1 NORM (reference nn_ops.h:300-304) */
	const float* freq_factors; /* host: n_rot / 2 floats (L.rope_freqs), or NULL */
} nnc_hip_prep;

/* The step just before the attention core, for one layer and a batch of
 * n_tok tokens at positions pos0 .. pos0 + n_tok - 1, on the device
 * (reference model.cpp:1616-1691): per-head RMSNorm of Q and K with their
 * gammas (reference nn_ops.cpp:590-632) and of V without gamma when v_norm
 * (reference nn_ops.cpp:558-588), RoPE of Q and K (reference
 * nn_ops.cpp:1830-1873), then K and V of token t into row (pos0 + t) % rows
 * of buffer `buf` (BF16 with nnc_f32_to_bf16's rounding, reference
 * runtime.h:106-113, or F32). q, K and V get the bits nnc's CPU step gives:
 * the norms take their sums in nnc's order, and the cos and sin of the
 * rotation angles come from the host's libm (the one nnc calls) on the same
 * fp32 angles; they are computed once per new (positions, RoPE setup) and
 * kept for the next layers.
 *   q [n_tok][n_head * head_dim] F32, device memory: normalised and rotated in
 *     place, ready for nnc_hip_attend_device;
 *   k, v [n_tok][n_kv * head_dim] F32, device memory: read only.
 * Asynchronous on the cache's stream.
 * NNC_ERR_INVALID_ARGUMENT: bad buffer index, NULL pointers, n_tok <= 0,
 * pos0 < 0, n_tok > rows, head counts <= 0, n_kv * head_dim not the buffer's
 * kv_dim, n_rot odd, negative or above head_dim, rope_mode not 0 or 1, a
 * non-positive freq_base with n_rot > 0.
 * NNC_ERR_UNSUPPORTED_MODEL: head_dim above 512. */
nnc_status nnc_hip_kv_prep_append_device(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, float* q,
                                         const float* k, const float* v, const nnc_hip_prep* prep);

/* Copies rows row0 .. row0 + n_rows - 1 of buffer `buf` (raw element bits)
 * to host memory and waits. Either output may be NULL. */
nnc_status nnc_hip_kv_read(nnc_hip_kv* kv, int32_t buf, int32_t row0, int32_t n_rows, void* k_out, void* v_out);

/* The attention core of attention_forward (reference model.cpp:1693-1761)
 * for one layer whose K/V live in buffer `buf`:
 *   q   [n_tok][n_head * head_dim] F32, host memory;
 *   out [n_tok][n_head * head_dim] F32, host memory, written when the call
 *       returns (the call waits for the stream).
 * Token t sits at position pos0 + t and attends to the keys of
 * model_attn_span(causal, window, pos0 + t, n_seq): n_seq is pos0 + n_tok for
 * a session, window is the layer's sliding window or 0. scale is
 * hparams.attention_scale (reference model.cpp:613-624). An empty span gives
 * zeros (the l == 0 rule of reference nn_ops.cpp:492).
 * Up to 16 tokens (an nnc session's forward pass, MODEL_PREFILL_BATCH,
 * reference model.h:330) run the split-K kernel with each token on the split
 * grid a one-token call gives it, so every token of such a batch gets the
 * bits of its one-token call (the decode == batch property of reference
 * tests.cpp:2631-2661 that MTP verification relies on). Larger batches run
 * the MFMA prefill kernel (BF16, head_dim 64, 128 or 256 with a group of 1,
 * 2, 4 or 8) or the tiled fp32-MFMA kernel (F32, and the other head shapes
 * with head_dim a multiple of 16), within tolerance, not bit-identical;
 * other shapes stay on the split-K kernels. Supported shapes: every even
 * head_dim up to 512 (as nnc, reference model.cpp:714) with a group
 * n_head / n_kv up to 16 and group * head_dim up to 8192.
 * NNC_ERR_INVALID_ARGUMENT: bad buffer index, NULL pointers, n_tok <= 0,
 * pos0 < 0, n_seq < 1, n_head not a multiple of n_kv, n_kv * head_dim not the
 * buffer's kv_dim.
 * NNC_ERR_CONTEXT_FULL: a key the batch needs lies outside what the buffer
 * can hold (a full buffer with pos0 + n_tok > rows, or a ring too small for
 * the window plus the batch).
 * NNC_ERR_UNSUPPORTED_MODEL: a head_dim or group outside the supported set,
 * or a BF16 buffer of 2 GiB or more. */
nnc_status nnc_hip_attend(nnc_hip_kv* kv, int32_t buf, const float* q, float* out, int32_t n_tok, int32_t pos0,
                          int32_t n_seq, int32_t window, bool causal, int32_t n_head, int32_t n_kv,
                          int32_t head_dim, float scale);

/* As nnc_hip_attend with q and out in device memory; asynchronous on the
 * cache's stream (wait with nnc_hip_kv_sync). */
nnc_status nnc_hip_attend_device(nnc_hip_kv* kv, int32_t buf, const float* q, float* out, int32_t n_tok,
                                 int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head,
                                 int32_t n_kv, int32_t head_dim, float scale);

/* Bytes of the fixed per-device scratch of nnc_hip_attend_device_noalloc
 * (split partials of decode and of tiled batches). */
#define NNC_HIP_NOALLOC_SCRATCH_BYTES (32u << 20)

/* As nnc_hip_attend_device, for callers that cannot allocate device memory:
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. No counterpart in the reference. The call allocates nothing
 * (no hipMalloc, hipFree or allocating library routine): the split kernels'
 * partials go to a fixed array of NNC_HIP_NOALLOC_SCRATCH_BYTES in each
 * device's memory, which the library holds until the process ends. Every
 * call on a GPU shares that GPU's array, and the calls are asynchronous: two
 * no-alloc calls on different caches of one GPU (each cache has its own
 * stream) overlap on the GPU and race on the array, even when one thread
 * issues them one after the other, so the caller must order them (wait for
 * the first, or make the second cache's stream wait on it); calls on one
 * cache are ordered on its stream and do not race. The array's device
 * address is looked up when the first cache on a device is created, so the
 * call itself loads nothing. Every launch of a call is planned before the
 * first is enqueued, so a refused call changes nothing.
 * NNC_ERR_INVALID_ARGUMENT: as nnc_hip_attend_device, and when the call's
 * partials would exceed the array (the message gives both sizes); one
 * decode token of Qwen3-4B at 32k context needs about 1 MiB, a 16-token
 * session batch about 16 MiB. */
nnc_status nnc_hip_attend_device_noalloc(nnc_hip_kv* kv, int32_t buf, const float* q, float* out, int32_t n_tok,
                                         int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head,
                                         int32_t n_kv, int32_t head_dim, float scale);

/* As nnc_hip_attend / nnc_hip_attend_device, then Qwen3.5's output gate:
 * out[i] *= 1 / (1 + exp(-gate[i])), with gate [n_tok][n_head * head_dim]
 * F32 in the same memory as q (reference model.cpp:1759-1760,
 * nn_ops.cpp:1731-1742 nnc_mul_sigmoid_f32), fused into the kernels' last
 * write. NNC_ERR_INVALID_ARGUMENT also for a NULL gate. */
nnc_status nnc_hip_attend_gated(nnc_hip_kv* kv, int32_t buf, const float* q, const float* gate, float* out,
                                int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal,
                                int32_t n_head, int32_t n_kv, int32_t head_dim, float scale);
nnc_status nnc_hip_attend_gated_device(nnc_hip_kv* kv, int32_t buf, const float* q, const float* gate, float* out,
                                       int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal,
                                       int32_t n_head, int32_t n_kv, int32_t head_dim, float scale);

/* The weight gemvs on either side of attention (QKV and output projections,
 * MLP, lm_head; reference model.cpp:1189-1210 picks one by tensor type):
 *   Y[n][r] = sum_k W[r][k] * X[n][k],  n < n_batch, r < rows, k < cols,
 * with X n_batch vectors of cols floats x_stride floats apart and Y n_batch
 * vectors of rows floats y_stride floats apart (n_batch == 1 is the decode
 * gemv). All pointers are device memory; the call is queued on the cache's
 * stream (`kv` is the execution context: its stream and scratch). Weights in
 * nnc's three layouts:
 *   nnc_hip_gemv_bf16  W BF16 row-major [rows][cols] (reference nn_ops.h:95-96,
 *                      :156-159 nnc_gemv_bf16w_f32x(_batch));
 *   nnc_hip_gemv_q8_0  split Q8_0: qs int8 [rows][cols], scales BF16
 *                      [rows][cols/32] (nn_ops.h:119-121, :161-164);
 *   nnc_hip_gemv_q4_s  split Q4_S: qs nibbles [rows][cols/2] (byte i of a
 *                      block holds elements i and i+16), scales and biases BF16
 *                      [rows][cols/32]; XSUM the per-32 block sums of each X
 *                      vector, xsum_stride apart (nnc_block_sums_f32), or NULL
 *                      to have them computed (nn_ops.h:138-142, :168-175).
 * rows, cols or n_batch of 0 is a no-op, as in the reference.
 * NNC_ERR_INVALID_ARGUMENT: NULL pointers, strides below cols / rows, W or X
 * not 16-byte aligned or x_stride not a multiple of 4.
 * NNC_ERR_UNSUPPORTED_MODEL: cols not a multiple of 32. */
nnc_status nnc_hip_gemv_bf16(nnc_hip_kv* kv, const void* W, const float* X, size_t x_stride, float* Y, size_t y_stride,
                             uint32_t rows, uint32_t cols, uint32_t n_batch);
nnc_status nnc_hip_gemv_q8_0(nnc_hip_kv* kv, const int8_t* qs, const uint16_t* scales, const float* X,
                             size_t x_stride, float* Y, size_t y_stride, uint32_t rows, uint32_t cols,
                             uint32_t n_batch);
nnc_status nnc_hip_gemv_q4_s(nnc_hip_kv* kv, const uint8_t* qs, const uint16_t* scales, const uint16_t* biases,
                             const float* X, size_t x_stride, const float* XSUM, size_t xsum_stride, float* Y,
                             size_t y_stride, uint32_t rows, uint32_t cols, uint32_t n_batch);

/* Several of the gemvs above over the same X in one launch: the QKV
 * projections (reference model.cpp:1596-1602, three gemv_batch calls on the
 * same normed input) or the FFN gate and up projections (:1816-1817). No
 * counterpart in nnc, which runs them one by one; every mats[m].y receives
 * exactly what the single-matrix call for that matrix writes (the same
 * kernels, the same sums per row). format is NNC_HIP_GEMV_BF16, _Q8_0 or
 * _Q4_S, n_mat 1 .. NNC_HIP_GEMV_MAX_GROUP, every matrix of cols columns in
 * that layout (scales for Q8_0 and Q4_S, biases for Q4_S, NULL otherwise);
 * XSUM as for nnc_hip_gemv_q4_s (ignored for other formats). One launch per
 * 16 vectors for the whole group when every matrix but the last has a
 * multiple of 16 rows (nnc's projections do), else one per matrix. Errors as
 * for the single-matrix calls, and NNC_ERR_INVALID_ARGUMENT for an unknown
 * format or n_mat out of range. */
enum
{
	NNC_HIP_GEMV_BF16 = 0,
	NNC_HIP_GEMV_Q8_0 = 1,
	NNC_HIP_GEMV_Q4_S = 2,
	NNC_HIP_GEMV_MAX_GROUP = 3
};
typedef struct nnc_hip_gemv_mat
{
	const void* w; /* BF16 W, Q8_0 qs or Q4_S nibbles [rows][...] */
	const uint16_t* scales; /* [rows][cols / 32] BF16 (Q8_0, Q4_S) */
	const uint16_t* biases; /* [rows][cols / 32] BF16 (Q4_S) */
	float* y; /* n_batch vectors of rows floats, y_stride apart */
	size_t y_stride;
	uint32_t rows;
} nnc_hip_gemv_mat;
nnc_status nnc_hip_gemv_group(nnc_hip_kv* kv, int32_t format, int32_t n_mat, const nnc_hip_gemv_mat* mats,
                              const float* X, size_t x_stride, const float* XSUM, size_t xsum_stride, uint32_t cols,
                              uint32_t n_batch);

/* Greedy decode's lm_head projection: the row of the largest element of
 * y = W x for a BF16 W [rows][cols] and one vector x, without writing y
 * (reference nn_ops.h:98-113, nn_ops.cpp:1055-1197 nnc_gemv_bf16w_argmax_f32x;
 * caller model_argmax, model.cpp:2181-2190). *index (host memory) receives
 * the smallest such row; NaN and -inf are never chosen, and 0 is returned
 * when no element is above -inf; when rows is not a multiple of 4, 0 also
 * when y[0] is NaN (the reference's fallback scans from y[0]); -1 when rows
 * or cols is 0. W and x are device memory; the call waits for the cache's
 * stream. Errors as nnc_hip_gemv_bf16; cols must also fit the one-vector
 * kernel (at most 15 872). */
nnc_status nnc_hip_gemv_bf16_argmax(nnc_hip_kv* kv, const void* W, const float* x, uint32_t rows, uint32_t cols,
                                    int32_t* index);

/* The same over logits already on the device (the quantised lm_head's
 * scan after its gemv, reference model.cpp:2192-2195): the first r with
 * y[r] > y[best] for every earlier best, starting from best = 0, i.e. the
 * smallest row of the largest value, NaN never chosen, and 0 when y[0] is
 * NaN or nothing is above -inf (also for n == 0). y is device memory; the
 * call waits for the cache's stream. */
nnc_status nnc_hip_argmax_f32(nnc_hip_kv* kv, const float* y, uint32_t n, int32_t* index);

/* Waits for all work queued on the cache's stream. */
nnc_status nnc_hip_kv_sync(nnc_hip_kv* kv);

/* The cache's hipStream_t, for callers that order their own work on it. */
void* nnc_hip_kv_stream(nnc_hip_kv* kv);

/* Fills n elements at device address dst with N(0,1) values from the
 * counter-based generator splitmix64 + Box-Muller (element i comes from
 * draws 2*(i/2) and 2*(i/2)+1 of the stream `seed`), then, when norm_dim > 0,
 * RMS-normalises each run of norm_dim elements (eps 1e-6), then stores them
 * as F32 (bf16 == false) or BF16 rounded to nearest even (bf16 == true).
 * Queued on `stream` (a hipStream_t; NULL is the null stream). This is the
 * synthetic-input generator of the benchmark and has no counterpart in the
 * reference. */
nnc_status nnc_hip_fill_normal(void* dst, uint64_t n, uint64_t seed, int32_t norm_dim, bool bf16, void* stream);

/* Detail of the most recent failure on the calling thread; never NULL. */
const char* nnc_hip_last_error(void);

/* A short description of `status` (the strings of nnc_status_string). */
const char* nnc_hip_status_string(nnc_status status);

#ifdef __cplusplus
}
#endif

#endif /* NNC_HIP_H */
