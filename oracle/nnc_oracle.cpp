// TEST INFRASTRUCTURE — the CPU oracle. Only tests/, the smoke check and
// bench.py's cpu_baseline leg may load liboracle.so; the product path (the
// HIP library under libllmcpu_amd/) never links, loads or calls it.
//
// A plain C++ restatement of nnc's attention hot path, written from the
// reference's behaviour, one function per reference routine:
//   orc_bf16_from_f32 / orc_f32_from_bf16  reference src/libnnc/runtime.h:97-113
//   orc_attn_block                         reference src/libnnc/nn_ops.cpp:326-459
//   orc_attn_merge                         reference src/libnnc/nn_ops.cpp:461-482
//   orc_attn_finish                        reference src/libnnc/nn_ops.cpp:484-499
//   orc_attn_span                          reference src/libnnc/model.cpp:2300-2316
//   orc_kv_rows / orc_max_rewind           reference src/libnnc/model.cpp:1936-1957
//   orc_attend_layer                       reference src/libnnc/model.cpp:1229-1317, 1693-1757
//   orc_rope / orc_rope_ff                 reference src/libnnc/nn_ops.cpp:1830-1873
//   orc_rmsnorm_groups                     reference src/libnnc/nn_ops.cpp:590-632 (gamma = 1)
//   orc_rmsnorm_gamma                      reference src/libnnc/nn_ops.cpp:590-632
//   orc_rmsnorm_plain                      reference src/libnnc/nn_ops.cpp:558-588
//   orc_prep_append                        reference src/libnnc/model.cpp:1616-1691 (per-head
//                                          Q/K/V norms, RoPE on Q and K, K/V append)
//   orc_mul_sigmoid                        reference src/libnnc/nn_ops.cpp:1731-1742 (Qwen3.5's
//                                          output gate, model.cpp:1759-1760)
//   orc_quantize_q8_0 / orc_quantize_q4_s  reference src/libnnc/nn_ops.cpp:1223-1290 (split
//                                          layouts, docs/design.md:141-193)
//   orc_block_sums                         reference src/libnnc/nn_ops.cpp:1305-1316
//   orc_gemv_bf16 / orc_gemv_q8_0 /        reference src/libnnc/nn_ops.cpp:1000-1053, 1352-1452,
//   orc_gemv_q4_s                          1610-1700 (the weight gemvs, single and batched;
//                                          model.cpp:1189-1210 picks one by tensor type)
//   orc_gemv_bf16_argmax                   nn_ops.cpp:1055-1197 (lm_head argmax, model.cpp:2181-2190)
//   orc_argmax_f32                         model.cpp:2192-2195 (the quantised lm_head's scan)
// and two checkers that are not restatements:
//   orc_textbook_attend   double-precision softmax attention per query, the
//                         scalar reference of reference src/appnnc/tests.cpp:2424-2446
//                         lifted to a whole layer (spans, GQA, ring rows);
//   orc_ref_fixture_attn_blocks  the input recipe of the reference's own
//                         test_nnc_attn_blocks (reference src/appnnc/tests.cpp:2450-2476):
//                         std::mt19937(7) and std::normal_distribution<float>.
//
// Arithmetic: fp32 with the reference's loop structure (scores per key for
// all heads of the group, the block's own max, exp, sum, then the V pass).
// exp is std::exp rather than the reference's AVX2 polynomial (relative
// difference below 3e-7, reference nn_ops.cpp:49-56).
#include "attend_dispatch.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <random>
#include <thread>
#include <limits>
#include <vector>

extern "C" {
void orc_attn_block(const float* q, size_t q_stride, const void* K, const void* V, int kv_bf16, size_t kv_stride,
                    size_t n_keys, size_t head_dim, size_t n_heads, float scale, float* scores, float* part);
void orc_attn_merge(float* acc, const float* part, size_t head_dim, size_t n_heads);
void orc_attn_finish(float* out, size_t out_stride, const float* acc, size_t head_dim, size_t n_heads);
}

namespace
{
	inline float bf16_to_f32(uint16_t v)
	{
		const uint32_t u = static_cast<uint32_t>(v) << 16;
		float f;
		std::memcpy(&f, &u, 4);
		return f;
	}

	inline uint16_t f32_to_bf16(float f)
	{
		uint32_t u;
		std::memcpy(&u, &f, 4);
		return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
	}

	template <typename T>
	inline float kv_at(const T* p, size_t i);
	template <>
	inline float kv_at<float>(const float* p, size_t i) { return p[i]; }
	template <>
	inline float kv_at<uint16_t>(const uint16_t* p, size_t i) { return bf16_to_f32(p[i]); }

	template <typename T>
	void block_t(const float* q, size_t q_stride, const T* K, const T* V, size_t kv_stride, size_t n_keys,
	             size_t hd, size_t n_heads, float scale, float* scores, float* part)
	{
		const size_t pw = orc::part_floats(hd);
		std::vector<float> krow(hd);
		// Scores: each key row is widened once and dotted with every head.
		for (size_t t = 0; t < n_keys; ++t)
		{
			const T* k = K + t * kv_stride;
			for (size_t i = 0; i < hd; ++i) krow[i] = kv_at(k, i);
			for (size_t h = 0; h < n_heads; ++h)
			{
				const float* qh = q + h * q_stride;
				float s = 0.0f;
				for (size_t i = 0; i < hd; ++i) s += qh[i] * krow[i];
				scores[h * n_keys + t] = s * scale;
			}
		}
		// Per head: the block's own max, the weights and their sum.
		for (size_t h = 0; h < n_heads; ++h)
		{
			float* s = scores + h * n_keys;
			float m = s[0];
			for (size_t t = 1; t < n_keys; ++t) m = std::max(m, s[t]);
			float l = 0.0f;
			for (size_t t = 0; t < n_keys; ++t)
			{
				s[t] = std::exp(s[t] - m);
				l += s[t];
			}
			part[h * pw + hd] = m;
			part[h * pw + hd + 1] = l;
		}
		// Weighted sum of V rows, the row outermost so it is read once.
		for (size_t h = 0; h < n_heads; ++h) std::fill(part + h * pw, part + h * pw + hd, 0.0f);
		for (size_t t = 0; t < n_keys; ++t)
		{
			const T* vr = V + t * kv_stride;
			for (size_t i = 0; i < hd; ++i) krow[i] = kv_at(vr, i);
			for (size_t h = 0; h < n_heads; ++h)
			{
				const float w = scores[h * n_keys + t];
				float* o = part + h * pw;
				for (size_t i = 0; i < hd; ++i) o[i] += w * krow[i];
			}
		}
	}

	// A plain fork-join pool: an even split of [0, n) over the threads, the
	// caller taking the first range (the split of reference nn_ops.cpp:960-969).
	struct thread_ops
	{
		int threads = 1;

		int n_threads() const { return threads; }

		void block(const float* q, size_t q_stride, const void* K, const void* V, bool bf16, size_t kv_stride,
		           size_t n_keys, size_t hd, size_t n_heads, float scale, float* scores, float* part) const
		{
			orc_attn_block(q, q_stride, K, V, bf16 ? 1 : 0, kv_stride, n_keys, hd, n_heads, scale, scores, part);
		}
		void merge(float* acc, const float* part, size_t hd, size_t n_heads) const
		{
			orc_attn_merge(acc, part, hd, n_heads);
		}
		void finish(float* out, size_t out_stride, const float* acc, size_t hd, size_t n_heads) const
		{
			orc_attn_finish(out, out_stride, acc, hd, n_heads);
		}

		void parallel_for(uint32_t n, void (*fn)(uint32_t, uint32_t, void*), void* user) const
		{
			if (n == 0) return;
			const uint32_t nt = std::min<uint32_t>(n, static_cast<uint32_t>(std::max(1, threads)));
			if (nt == 1)
			{
				fn(0, n, user);
				return;
			}
			auto range = [&](uint32_t tid, uint32_t& a, uint32_t& b)
			{
				const uint32_t per = n / nt, rem = n % nt;
				a = tid * per + std::min(tid, rem);
				b = a + per + (tid < rem ? 1u : 0u);
			};
			std::vector<std::thread> pool;
			for (uint32_t tid = 1; tid < nt; ++tid)
			{
				uint32_t a, b;
				range(tid, a, b);
				pool.emplace_back([=] { if (a < b) fn(a, b, user); });
			}
			uint32_t a, b;
			range(0, a, b);
			if (a < b) fn(a, b, user);
			for (auto& t : pool) t.join();
		}
	};
}

extern "C" {

uint16_t orc_bf16_from_f32(float f) { return f32_to_bf16(f); }
float orc_f32_from_bf16(uint16_t v) { return bf16_to_f32(v); }

void orc_bf16_round(const float* x, uint16_t* y, size_t n)
{
	for (size_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
}

void orc_attn_block(const float* q, size_t q_stride, const void* K, const void* V, int kv_bf16, size_t kv_stride,
                    size_t n_keys, size_t head_dim, size_t n_heads, float scale, float* scores, float* part)
{
	if (n_keys == 0 || n_heads == 0) return; // reference nn_ops.cpp:452
	if (kv_bf16)
		block_t(q, q_stride, static_cast<const uint16_t*>(K), static_cast<const uint16_t*>(V), kv_stride, n_keys,
		        head_dim, n_heads, scale, scores, part);
	else
		block_t(q, q_stride, static_cast<const float*>(K), static_cast<const float*>(V), kv_stride, n_keys, head_dim,
		        n_heads, scale, scores, part);
}

void orc_attn_merge(float* acc, const float* part, size_t head_dim, size_t n_heads)
{
	const size_t pw = orc::part_floats(head_dim);
	for (size_t h = 0; h < n_heads; ++h)
	{
		float* a = acc + h * pw;
		const float* b = part + h * pw;
		const float m = std::max(a[head_dim], b[head_dim]);
		const float ca = std::exp(a[head_dim] - m);
		const float cb = std::exp(b[head_dim] - m);
		for (size_t i = 0; i < head_dim; ++i) a[i] = a[i] * ca + b[i] * cb;
		a[head_dim] = m;
		a[head_dim + 1] = a[head_dim + 1] * ca + b[head_dim + 1] * cb;
	}
}

void orc_attn_finish(float* out, size_t out_stride, const float* acc, size_t head_dim, size_t n_heads)
{
	const size_t pw = orc::part_floats(head_dim);
	for (size_t h = 0; h < n_heads; ++h)
	{
		const float* a = acc + h * pw;
		const float l = a[head_dim + 1];
		const float inv = l > 0.0f ? 1.0f / l : 0.0f; // l == 0 gives 0 (reference nn_ops.cpp:492)
		for (size_t i = 0; i < head_dim; ++i) out[h * out_stride + i] = a[i] * inv;
	}
}

void orc_attn_span(int causal, int window, int pos, int n_seq, int* first, int* last)
{
	orc::attn_span(causal != 0, window, pos, n_seq, first, last);
}

int orc_kv_rows(int n_ctx, int window, int n_batch) { return orc::kv_rows(n_ctx, window, n_batch); }

// How far below the highest written position a ring lets a cache go back
// (reference model.cpp:1949, max_rewind = rows - window).
int orc_max_rewind(int rows, int window) { return rows - window; }

// One layer's attention over nnc's K/V layout with this file's kernels.
// Returns 0, or -1 for arguments the reference would never pass.
int orc_attend_layer(const float* q, float* out, const void* K, const void* V, int kv_bf16, int rows, int n_tok,
                     int pos0, int n_seq, int window, int causal, int n_head, int n_kv, int head_dim, float scale,
                     int n_threads)
{
	if (n_tok <= 0 || n_kv <= 0 || n_head % n_kv != 0 || head_dim <= 0 || rows <= 0) return -1;
	orc::attend_args a{q,     out,   static_cast<const uint8_t*>(K), static_cast<const uint8_t*>(V), kv_bf16 != 0,
	                   rows,  n_tok, pos0, n_seq, window, causal != 0, n_head, n_kv, head_dim, scale};
	thread_ops ops;
	ops.threads = std::max(1, std::min(n_threads, 64));
	static thread_local orc::attend_scratch scratch;
	orc::attend_runner<thread_ops> runner(ops, a, scratch);
	runner.run();
	return 0;
}

// Double-precision softmax attention of every query head over its span, the
// same addressing as the op (row k % rows, KV head h / group).
void orc_textbook_attend(const float* q, float* out, const void* K, const void* V, int kv_bf16, int rows, int n_tok,
                         int pos0, int n_seq, int window, int causal, int n_head, int n_kv, int head_dim, float scale)
{
	const int group = n_head / n_kv;
	const size_t hd = static_cast<size_t>(head_dim), kv_dim = static_cast<size_t>(n_kv) * hd;
	auto at = [&](const void* base, size_t row, size_t i) -> double
	{
		const size_t idx = row * kv_dim + i;
		return kv_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(base)[idx]) : static_cast<const float*>(base)[idx];
	};
	std::vector<double> s, o(hd);
	for (int t = 0; t < n_tok; ++t)
	{
		int first, last;
		orc::attn_span(causal != 0, window, pos0 + t, n_seq, &first, &last);
		for (int h = 0; h < n_head; ++h)
		{
			const float* qh = q + (static_cast<size_t>(t) * n_head + h) * hd;
			const size_t koff = static_cast<size_t>(h / group) * hd;
			float* oh = out + (static_cast<size_t>(t) * n_head + h) * hd;
			if (last < first)
			{
				std::fill(oh, oh + hd, 0.0f);
				continue;
			}
			s.assign(static_cast<size_t>(last - first + 1), 0.0);
			double m = -1e300;
			for (int k = first; k <= last; ++k)
			{
				const size_t row = static_cast<size_t>(k % rows);
				double d = 0.0;
				for (size_t i = 0; i < hd; ++i) d += static_cast<double>(qh[i]) * at(K, row, koff + i);
				s[k - first] = d * scale;
				m = std::max(m, s[k - first]);
			}
			double sum = 0.0;
			for (double& v : s) sum += (v = std::exp(v - m));
			std::fill(o.begin(), o.end(), 0.0);
			for (int k = first; k <= last; ++k)
			{
				const size_t row = static_cast<size_t>(k % rows);
				const double w = s[k - first];
				for (size_t i = 0; i < hd; ++i) o[i] += w * at(V, row, koff + i);
			}
			for (size_t i = 0; i < hd; ++i) oh[i] = static_cast<float>(o[i] / sum);
		}
	}
}

// Rotary embedding of n_heads vectors of head_dim floats at position pos:
// angle_i = pos * base^(-2i/n_rot) (divided by freq_factors[i] when given),
// the per-step ratio accumulated in fp32; mode 0 (NEOX) pairs lanes i and
// i + n_rot/2, mode 1 (NORM) lanes 2i and 2i+1; lanes past n_rot pass through.
void orc_rope_ff(float* x, int n_heads, int head_dim, int n_rot, float pos, float base, int mode, const float* ff)
{
	if (n_rot <= 0) return;
	const int half = n_rot / 2;
	std::vector<float> c(half), s(half);
	const float ratio = std::pow(base, -2.0f / static_cast<float>(n_rot));
	float inv = 1.0f;
	for (int i = 0; i < half; ++i)
	{
		float th = pos * inv;
		if (ff) th /= ff[i];
		c[i] = std::cos(th);
		s[i] = std::sin(th);
		inv *= ratio;
	}
	const int stride = mode == 0 ? 1 : 2;
	const int partner = mode == 0 ? half : 1;
	for (int h = 0; h < n_heads; ++h)
	{
		float* xh = x + static_cast<size_t>(h) * head_dim;
		for (int i = 0; i < half; ++i)
		{
			float* p = xh + i * stride;
			const float a = p[0], b = p[partner];
			// The reference's build contracts each of the two expressions into
			// one fused multiply-add, the first product fused and the second
			// rounded (its -ffast-math build, reference CMakeLists.txt:66-76);
			// bit for bit against it in tests/test_oracle.py.
			const float sb = s[i] * b, cb = c[i] * b;
			p[0] = std::fma(c[i], a, -sb);
			p[partner] = std::fma(s[i], a, cb);
		}
	}
}

void orc_rope(float* x, int n_heads, int head_dim, int n_rot, float pos, float base, int mode)
{
	orc_rope_ff(x, n_heads, head_dim, n_rot, pos, base, mode, nullptr);
}

// The sum of squares of dim floats as the reference's AVX2 loop takes it
// (reference nn_ops.cpp:562-575, :600-613): eight fp32 fused multiply-add
// chains over x[l], x[l + 8], ... for the full runs of eight, their sum in
// hsum_ymm's order ((c0 + c4) + (c1 + c5)) + ((c2 + c6) + (c3 + c7))
// (reference nn_ops.cpp:28-36), then the tail in double.
void orc_rmsnorm_gamma(float* x, size_t n_groups, size_t dim, const float* gamma, float eps);

static double rms_sum_squares(const float* x, size_t dim)
{
	double s2 = 0.0;
	size_t i = 0;
	if (dim >= 8)
	{
		float c[8] = {};
		for (; i + 8 <= dim; i += 8)
			for (int l = 0; l < 8; ++l) c[l] = std::fma(x[i + l], x[i + l], c[l]);
		const float hs = ((c[0] + c[4]) + (c[1] + c[5])) + ((c[2] + c[6]) + (c[3] + c[7]));
		s2 = static_cast<double>(hs);
	}
	for (; i < dim; ++i) s2 += static_cast<double>(x[i]) * x[i];
	return s2;
}

// RMSNorm of n_groups vectors of dim floats, in place, gamma = 1
// (nnc_rmsnorm_gamma_multi_f32 with unit gamma).
void orc_rmsnorm_groups(float* x, size_t n_groups, size_t dim, float eps)
{
	orc_rmsnorm_gamma(x, n_groups, dim, nullptr, eps);
}

// RMSNorm with a learned gamma (NULL = 1), in place: scale = 1 / sqrt(sum *
// (1/dim as fp32) + eps) in double, rounded to fp32; y = (x * gamma) * scale,
// the order the reference's -ffast-math build multiplies in (bit for bit
// against it in tests/test_oracle.py).
void orc_rmsnorm_gamma(float* x, size_t n_groups, size_t dim, const float* gamma, float eps)
{
	const float inv_dim = 1.0f / static_cast<float>(dim);
	for (size_t g = 0; g < n_groups; ++g)
	{
		float* xg = x + g * dim;
		const double s2 = rms_sum_squares(xg, dim);
		const float r = static_cast<float>(1.0 / std::sqrt(s2 * inv_dim + eps));
		for (size_t i = 0; i < dim; ++i) xg[i] = (xg[i] * (gamma ? gamma[i] : 1.0f)) * r;
	}
}

// RMSNorm without gamma, in place: scale = 1 / sqrt(sum / dim + eps) in
// double, rounded to fp32; y = x * scale.
void orc_rmsnorm_plain(float* x, size_t n_groups, size_t dim, float eps)
{
	for (size_t g = 0; g < n_groups; ++g)
	{
		float* xg = x + g * dim;
		const double s2 = rms_sum_squares(xg, dim);
		const float r = static_cast<float>(1.0 / std::sqrt(s2 / static_cast<double>(dim) + eps));
		for (size_t i = 0; i < dim; ++i) xg[i] *= r;
	}
}

// y[i] *= sigmoid(g[i]): in runs of eight, y * (1 / (1 + exp(-g))); the tail
// past the last full run as y / (1 + exp(-g)).
void orc_mul_sigmoid(float* y, const float* g, size_t n)
{
	size_t i = 0;
	for (; i + 8 <= n; ++i) y[i] = y[i] * (1.0f / (1.0f + std::exp(-g[i])));
	for (; i < n; ++i) y[i] /= 1.0f + std::exp(-g[i]);
}

// Q8_0 split layout from fp32, one 32-element block at a time: the block's
// absmax / 127 rounded to BF16 is the scale; q = round-to-nearest-even of
// w / scale (w * (1 / scale)), clamped to [-127, 127]; a zero block has
// scale 0 and q 0. The reference is built with -ffast-math (reference
// CMakeLists.txt:66-76), which turns the division by the constant 127 into a
// multiplication by its fp32 reciprocal; so does this restatement.
void orc_quantize_q8_0(const float* src, int8_t* qs, uint16_t* scales, size_t n)
{
	for (size_t b = 0; b < n; b += 32)
	{
		float amax = 0.0f;
		for (size_t k = 0; k < 32; ++k) amax = std::max(amax, std::fabs(src[b + k]));
		const uint16_t sb = f32_to_bf16(amax * (1.0f / 127.0f));
		const float scale = bf16_to_f32(sb);
		scales[b / 32] = sb;
		const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
		for (size_t k = 0; k < 32; ++k)
		{
			const long q = std::lrintf(src[b + k] * inv);
			qs[b + k] = static_cast<int8_t>(std::min(127L, std::max(-127L, q)));
		}
	}
}

// Q4_S split layout from fp32: per 32-element block scale = (max - min) / 15
// and bias = min, both rounded to BF16 before use; q = rne((w - bias) / scale)
// clamped to [0, 15]; byte i of a block holds element i (low nibble) and
// element i + 16 (high nibble). (max - min) / 15 is evaluated as
// (max - min) * (1 / 15), as the reference's -ffast-math build does.
void orc_quantize_q4_s(const float* src, uint8_t* qs, uint16_t* scales, uint16_t* biases, size_t n)
{
	for (size_t b = 0; b < n; b += 32)
	{
		float lo = src[b], hi = src[b];
		for (size_t k = 1; k < 32; ++k)
		{
			lo = std::min(lo, src[b + k]);
			hi = std::max(hi, src[b + k]);
		}
		const uint16_t sb = f32_to_bf16((hi - lo) * (1.0f / 15.0f)), bb = f32_to_bf16(lo);
		const float scale = bf16_to_f32(sb), bias = bf16_to_f32(bb);
		scales[b / 32] = sb;
		biases[b / 32] = bb;
		const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
		for (size_t k = 0; k < 16; ++k)
		{
			const long q0 = std::min(15L, std::max(0L, std::lrintf((src[b + k] - bias) * inv)));
			const long q1 = std::min(15L, std::max(0L, std::lrintf((src[b + k + 16] - bias) * inv)));
			qs[b / 2 + k] = static_cast<uint8_t>(q0 | (q1 << 4));
		}
	}
}

// out[b] = sum of x[32 b .. 32 b + 31] in fp32, in the order the
// reference's -ffast-math build evaluates its eight-lane sums: lane j is
// (x[j] + x[8 + j]) + (x[16 + j] + x[24 + j]), then the lanes pairwise as
// its horizontal sum does (reference nn_ops.cpp:27-36).
void orc_block_sums(const float* x, float* out, size_t n)
{
	for (size_t b = 0; b < n; b += 32)
	{
		float lane[8];
		for (int j = 0; j < 8; ++j) lane[j] = (x[b + j] + x[b + 8 + j]) + (x[b + 16 + j] + x[b + 24 + j]);
		out[b / 32] = ((lane[0] + lane[4]) + (lane[1] + lane[5])) + ((lane[2] + lane[6]) + (lane[3] + lane[7]));
	}
}

// y[n][r] = sum_k W[r][k] x[n][k] with W BF16 row-major [rows][cols]; fp32
// products summed in fp32 in column order.
void orc_gemv_bf16(const uint16_t* W, const float* X, size_t x_stride, float* Y, size_t y_stride, uint32_t rows,
                   uint32_t cols, uint32_t n_batch)
{
	for (uint32_t n = 0; n < n_batch; ++n)
		for (uint32_t r = 0; r < rows; ++r)
		{
			const uint16_t* w = W + static_cast<size_t>(r) * cols;
			const float* x = X + n * x_stride;
			float s = 0.0f;
			for (uint32_t k = 0; k < cols; ++k) s += bf16_to_f32(w[k]) * x[k];
			Y[n * y_stride + r] = s;
		}
}

// argmax_r y[r] of the BF16 gemv above (reference nn_ops.cpp:1055-1197,
// nnc_gemv_bf16w_argmax_f32x): -1 for an empty matrix; when rows is a multiple
// of 4 and cols of 8 (its fast paths, threaded or not) the first row whose
// value is above every earlier one, starting from -inf, else 0; otherwise
// (its fallback) the first row above every earlier one starting from y[0].
int orc_gemv_bf16_argmax(const uint16_t* W, const float* x, uint32_t rows, uint32_t cols)
{
	if (rows == 0 || cols == 0) return -1;
	std::vector<float> y(rows);
	orc_gemv_bf16(W, x, cols, y.data(), rows, rows, cols, 1);
	const bool fast = rows % 4 == 0 && cols % 8 == 0;
	int best = 0;
	float bv = fast ? -std::numeric_limits<float>::infinity() : y[0];
	for (uint32_t r = fast ? 0 : 1; r < rows; ++r)
		if (y[r] > bv)
		{
			bv = y[r];
			best = static_cast<int>(r);
		}
	return best;
}

// The quantised lm_head's argmax over its logits (reference
// model.cpp:2192-2195): best starts at 0, and a row replaces it when its value
// is strictly larger.
int orc_argmax_f32(const float* y, uint32_t n)
{
	int best = 0;
	for (uint32_t r = 1; r < n; ++r)
		if (y[r] > y[best]) best = static_cast<int>(r);
	return best;
}

// Q8_0 split layout: y = sum over blocks of scale_b * (sum_{k in b} q_k x_k).
void orc_gemv_q8_0(const int8_t* qs, const uint16_t* scales, const float* X, size_t x_stride, float* Y,
                   size_t y_stride, uint32_t rows, uint32_t cols, uint32_t n_batch)
{
	const uint32_t nb = cols / 32;
	for (uint32_t n = 0; n < n_batch; ++n)
		for (uint32_t r = 0; r < rows; ++r)
		{
			const float* x = X + n * x_stride;
			float s = 0.0f;
			for (uint32_t b = 0; b < nb; ++b)
			{
				const int8_t* q = qs + static_cast<size_t>(r) * cols + 32 * b;
				float d = 0.0f;
				for (int k = 0; k < 32; ++k) d += static_cast<float>(q[k]) * x[32 * b + k];
				s += bf16_to_f32(scales[static_cast<size_t>(r) * nb + b]) * d;
			}
			Y[n * y_stride + r] = s;
		}
}

// Q4_S split layout: y = sum_b scale_b * (sum_{k in b} q_k x_k) + sum_b
// bias_b * S_b, S_b = xsum[b] (the block sums of x).
void orc_gemv_q4_s(const uint8_t* qs, const uint16_t* scales, const uint16_t* biases, const float* X,
                   size_t x_stride, const float* XSUM, size_t xsum_stride, float* Y, size_t y_stride, uint32_t rows,
                   uint32_t cols, uint32_t n_batch)
{
	const uint32_t nb = cols / 32;
	for (uint32_t n = 0; n < n_batch; ++n)
		for (uint32_t r = 0; r < rows; ++r)
		{
			const float* x = X + n * x_stride;
			float s = 0.0f, t = 0.0f;
			for (uint32_t b = 0; b < nb; ++b)
			{
				const uint8_t* q = qs + (static_cast<size_t>(r) * cols + 32 * b) / 2;
				float d = 0.0f;
				for (int k = 0; k < 16; ++k)
				{
					d += static_cast<float>(q[k] & 15) * x[32 * b + k];
					d += static_cast<float>(q[k] >> 4) * x[32 * b + 16 + k];
				}
				s += bf16_to_f32(scales[static_cast<size_t>(r) * nb + b]) * d;
				t += bf16_to_f32(biases[static_cast<size_t>(r) * nb + b]) * XSUM[n * xsum_stride + b];
			}
			Y[n * y_stride + r] = s + t;
		}
}

// The step before the attention core, in the reference's order: per-head
// RMSNorm of Q (q_gamma) and K (k_gamma) when given, of V without gamma when
// v_norm (Gemma 4), RoPE of Q and K at position (pos0 + t) * pos_scale, then
// K and V of token t to row (pos0 + t) % rows of the buffers (BF16 with
// round-to-nearest-even, or F32). q, k and v ([n_tok][heads * head_dim]) are
// updated in place, as the reference updates its scratch rows.
void orc_prep_append(float* q, float* k, float* v, int n_tok, int n_head, int n_kv, int head_dim,
                     const float* q_gamma, const float* k_gamma, int v_norm, float eps, int n_rot, float base,
                     float pos_scale, int mode, const float* ff, int pos0, int rows, int kv_bf16, void* K, void* V)
{
	const size_t q_dim = static_cast<size_t>(n_head) * head_dim, kv_dim = static_cast<size_t>(n_kv) * head_dim;
	if (q_gamma) orc_rmsnorm_gamma(q, static_cast<size_t>(n_tok) * n_head, head_dim, q_gamma, eps);
	if (k_gamma) orc_rmsnorm_gamma(k, static_cast<size_t>(n_tok) * n_kv, head_dim, k_gamma, eps);
	if (v_norm) orc_rmsnorm_plain(v, static_cast<size_t>(n_tok) * n_kv, head_dim, eps);
	for (int t = 0; t < n_tok; ++t)
	{
		const float rpos = static_cast<float>(pos0 + t) * pos_scale;
		orc_rope_ff(q + t * q_dim, n_head, head_dim, n_rot, rpos, base, mode, ff);
		orc_rope_ff(k + t * kv_dim, n_kv, head_dim, n_rot, rpos, base, mode, ff);
	}
	for (int t = 0; t < n_tok; ++t)
	{
		const size_t row = static_cast<size_t>((pos0 + t) % rows) * kv_dim;
		for (size_t i = 0; i < kv_dim; ++i)
		{
			if (kv_bf16)
			{
				static_cast<uint16_t*>(K)[row + i] = f32_to_bf16(k[t * kv_dim + i]);
				static_cast<uint16_t*>(V)[row + i] = f32_to_bf16(v[t * kv_dim + i]);
			}
			else
			{
				static_cast<float*>(K)[row + i] = k[t * kv_dim + i];
				static_cast<float*>(V)[row + i] = v[t * kv_dim + i];
			}
		}
	}
}

// The inputs of the reference's test_nnc_attn_blocks case `which` (0..3 in
// its loop order: F32 hd 64, F32 hd 36, BF16 hd 64, BF16 hd 36): one
// std::mt19937(7) stream, q ~ N(0,1), K ~ 2 N(0,1), V ~ N(0,1) per case, with
// group 3, n_kv 2, 600 keys. Writes q [3*hd], K and V [600 * 2*hd] as F32.
// Returns hd, or -1 for a bad index.
int orc_ref_fixture_attn_blocks(int which, float* q, float* K, float* V)
{
	if (which < 0 || which > 3) return -1;
	std::mt19937 rng(7);
	std::normal_distribution<float> nd(0.0f, 1.0f);
	int hd_out = -1;
	int idx = 0;
	for (const bool bf16 : {false, true})
		for (const int hd : {64, 36})
		{
			(void)bf16;
			const size_t group = 3, n_kv = 2, kv_stride = n_kv * hd, n_keys = 600;
			std::vector<float> qq(group * hd), KK(n_keys * kv_stride), VV(n_keys * kv_stride);
			for (float& x : qq) x = nd(rng);
			for (float& x : KK) x = 2.0f * nd(rng);
			for (float& x : VV) x = nd(rng);
			if (idx == which)
			{
				std::memcpy(q, qq.data(), qq.size() * 4);
				std::memcpy(K, KK.data(), KK.size() * 4);
				std::memcpy(V, VV.data(), VV.size() * 4);
				hd_out = hd;
			}
			++idx;
		}
	return hd_out;
}

} // extern "C"
