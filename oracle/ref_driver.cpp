// TEST INFRASTRUCTURE — a C-ABI driver over the reference's own compiled
// code. oracle/Makefile builds it, together with the reference's sources
// compiled where they lie under /root/reference/src/libnnc, into
// oracle/_ref/libnnc_ref.so. Tests use it to pin the oracle against the real
// nnc kernels, tests/golden/make_golden.py writes fixtures from it, and
// bench.py's cpu_baseline leg times it. The product never loads it.
//
// What is the reference's and what is not:
//   ref_attn_block / ref_attn_merge / ref_attn_finish  call nnc_attn_block /
//       nnc_attn_merge / nnc_attn_finish (reference nn_ops.h:53-61);
//   ref_attn_span    calls model_attn_span (reference model.h:364);
//   ref_bf16_from_f32 calls nnc_f32_to_bf16 (reference runtime.h:106-113);
//   ref_rope         calls nnc_rope_f32 (reference nn_ops.h:306);
//   ref_rope_ff      calls nnc_rope_f32 with frequency factors;
//   ref_rmsnorm_groups / ref_rmsnorm_gamma call nnc_rmsnorm_gamma_multi_f32
//       (reference nn_ops.h:79), ref_rmsnorm_plain calls nnc_rmsnorm_f32
//       (reference nn_ops.h:73);
//   ref_mul_sigmoid  calls nnc_mul_sigmoid_f32 (reference nn_ops.h:248);
//   ref_quantize_q8_0 / ref_quantize_q4_s / ref_block_sums / ref_gemv_bf16 /
//       ref_gemv_bf16_argmax / ref_gemv_q8_0 / ref_gemv_q4_s call
//       nnc_gemv_bf16w_argmax_f32x, nnc_quantize_f32_to_q8_0,
//       nnc_quantize_f32_to_q4_s, nnc_block_sums_f32 and the batched gemvs
//       (reference nn_ops.h:119-180, 193-205; the JIT kernels behind them);
//   ref_set_threads / ref_threads call nnc_set_num_threads / nnc_num_threads
//       (reference nnc.h:104-105);
//   ref_attend_layer drives nnc_attn_block/merge/finish through the reference's
//       worker pool (nnc_parallel_for, reference nn_ops.h:15) with this
//       repository's restatement of the dispatch of model.cpp:1229-1317 and
//       1693-1757 (oracle/attend_dispatch.h): attention_forward itself sits in
//       an anonymous namespace and cannot be called from outside model.cpp.
#include "attend_dispatch.h"

#include "model.h"
#include "nn_ops.h"
#include "nnc.h"
#include "runtime.h"

#include <vector>

namespace
{
	struct ref_ops
	{
		int n_threads() const { return nnc_num_threads(); }

		void block(const float* q, size_t q_stride, const void* K, const void* V, bool bf16, size_t kv_stride,
		           size_t n_keys, size_t hd, size_t n_heads, float scale, float* scores, float* part) const
		{
			nnc_attn_block(q, q_stride, K, V, bf16, kv_stride, n_keys, hd, n_heads, scale, scores, part);
		}
		void merge(float* acc, const float* part, size_t hd, size_t n_heads) const
		{
			nnc_attn_merge(acc, part, hd, n_heads);
		}
		void finish(float* out, size_t out_stride, const float* acc, size_t hd, size_t n_heads) const
		{
			nnc_attn_finish(out, out_stride, acc, hd, n_heads);
		}
		void parallel_for(uint32_t n, void (*fn)(uint32_t, uint32_t, void*), void* user) const
		{
			nnc_parallel_for(n, fn, user);
		}
	};
}

extern "C" {

void ref_attn_block(const float* q, size_t q_stride, const void* K, const void* V, int kv_bf16, size_t kv_stride,
                    size_t n_keys, size_t head_dim, size_t n_heads, float scale, float* scores, float* part)
{
	nnc_attn_block(q, q_stride, K, V, kv_bf16 != 0, kv_stride, n_keys, head_dim, n_heads, scale, scores, part);
}

void ref_attn_merge(float* acc, const float* part, size_t head_dim, size_t n_heads)
{
	nnc_attn_merge(acc, part, head_dim, n_heads);
}

void ref_attn_finish(float* out, size_t out_stride, const float* acc, size_t head_dim, size_t n_heads)
{
	nnc_attn_finish(out, out_stride, acc, head_dim, n_heads);
}

void ref_attn_span(int causal, int window, int pos, int n_seq, int* first, int* last)
{
	model_attn_span(causal != 0, window, pos, n_seq, first, last);
}

uint16_t ref_bf16_from_f32(float f) { return nnc_f32_to_bf16(f); }

void ref_bf16_round(const float* x, uint16_t* y, size_t n)
{
	for (size_t i = 0; i < n; ++i) y[i] = nnc_f32_to_bf16(x[i]);
}

void ref_rope(float* x, int n_heads, int head_dim, int n_rot, float pos, float base, int mode)
{
	nnc_rope_f32(x, static_cast<uint32_t>(n_heads), static_cast<uint32_t>(head_dim), static_cast<uint32_t>(n_rot), pos,
	             base, mode == 0 ? NNC_ROPE_NEOX : NNC_ROPE_NORM, nullptr);
}

void ref_rmsnorm_groups(float* x, size_t n_groups, size_t dim, float eps)
{
	std::vector<float> gamma(dim, 1.0f);
	nnc_rmsnorm_gamma_multi_f32(x, x, n_groups, dim, gamma.data(), eps);
}

void ref_rope_ff(float* x, int n_heads, int head_dim, int n_rot, float pos, float base, int mode, const float* ff)
{
	nnc_rope_f32(x, static_cast<uint32_t>(n_heads), static_cast<uint32_t>(head_dim), static_cast<uint32_t>(n_rot), pos,
	             base, mode == 0 ? NNC_ROPE_NEOX : NNC_ROPE_NORM, ff);
}

void ref_rmsnorm_gamma(float* x, size_t n_groups, size_t dim, const float* gamma, float eps)
{
	nnc_rmsnorm_gamma_multi_f32(x, x, n_groups, dim, gamma, eps);
}

void ref_rmsnorm_plain(float* x, size_t n_groups, size_t dim, float eps)
{
	for (size_t g = 0; g < n_groups; ++g) nnc_rmsnorm_f32(x + g * dim, x + g * dim, dim, eps);
}

void ref_mul_sigmoid(float* y, const float* g, size_t n) { nnc_mul_sigmoid_f32(y, g, n); }

void ref_quantize_q8_0(const float* src, int8_t* qs, uint16_t* scales, size_t n)
{
	nnc_quantize_f32_to_q8_0(src, qs, scales, n);
}

void ref_quantize_q4_s(const float* src, uint8_t* qs, uint16_t* scales, uint16_t* biases, size_t n)
{
	nnc_quantize_f32_to_q4_s(src, qs, scales, biases, n);
}

void ref_block_sums(const float* x, float* out, size_t n) { nnc_block_sums_f32(x, out, n); }

void ref_gemv_bf16(const uint16_t* W, const float* X, size_t x_stride, float* Y, size_t y_stride, uint32_t rows,
                   uint32_t cols, uint32_t n_batch)
{
	nnc_gemv_bf16w_f32x_batch(W, X, x_stride, Y, y_stride, rows, cols, n_batch);
}

int ref_gemv_bf16_argmax(const uint16_t* W, const float* x, uint32_t rows, uint32_t cols)
{
	return nnc_gemv_bf16w_argmax_f32x(W, x, rows, cols);
}

void ref_gemv_q8_0(const int8_t* qs, const uint16_t* scales, const float* X, size_t x_stride, float* Y,
                   size_t y_stride, uint32_t rows, uint32_t cols, uint32_t n_batch)
{
	nnc_gemv_q8_0_f32x_batch(qs, scales, X, x_stride, Y, y_stride, rows, cols, n_batch);
}

void ref_gemv_q4_s(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const float* X,
                   size_t x_stride, const float* XSUM, size_t xsum_stride, float* Y, size_t y_stride, uint32_t rows,
                   uint32_t cols, uint32_t n_batch)
{
	nnc_gemv_q4_s_f32x_batch(qs, scales, biases, X, x_stride, XSUM, xsum_stride, Y, y_stride, rows, cols, n_batch);
}

void ref_set_threads(int n) { nnc_set_num_threads(n); }
int ref_threads(void) { return nnc_num_threads(); }

int ref_attend_layer(const float* q, float* out, const void* K, const void* V, int kv_bf16, int rows, int n_tok,
                     int pos0, int n_seq, int window, int causal, int n_head, int n_kv, int head_dim, float scale)
{
	if (n_tok <= 0 || n_kv <= 0 || n_head % n_kv != 0 || head_dim <= 0 || rows <= 0) return -1;
	orc::attend_args a{q,     out,   static_cast<const uint8_t*>(K), static_cast<const uint8_t*>(V), kv_bf16 != 0,
	                   rows,  n_tok, pos0, n_seq, window, causal != 0, n_head, n_kv, head_dim, scale};
	static orc::attend_scratch scratch;
	ref_ops ops;
	orc::attend_runner<ref_ops> runner(ops, a, scratch);
	runner.run();
	return 0;
}

} // extern "C"
