// Split-K attention for the head shapes the MFMA kernels do not take: any
// even head_dim up to 512 and any query-head group with group * head_dim up
// to 8192 (nnc runs every even head_dim up to 512, reference
// src/libnnc/model.cpp:714 and nn_ops.cpp:1841; its block test uses 36,
// src/appnnc/tests.cpp:2450-2497), BF16 or F32 K/V.
//
// Grid: (split, KV head, token); a work-group of 256 threads takes one
// token's keys in one absolute-aligned split of split_keys keys (a multiple
// of 256, nnc's block size) for the `group` query heads of one KV head:
//   q       the group's rows, pre-scaled into log2 units, staged in LDS;
//   scores  thread t takes key c0 + t of each 256-key chunk and forms the
//           group's dot products over head_dim in fp32 (BF16 widened by a
//           16-bit shift), in ascending element order;
//   softmax per head: the chunk max, then the running (m, l) of the split
//           and O's rescale, reductions in a fixed lane order;
//   O       thread t owns outputs t, t + 256, ... of the group's
//           group * head_dim and adds the chunk's keys in ascending order.
// The split's partial (o, m, l) goes to the decode partials in the split-K
// layout ([token][KV head][split][group][head_dim + 4]) and the ordered merge
// kernel below writes o * (1 / l) (0 when l == 0, reference
// nn_ops.cpp:492); one split writes o * (1 / l) directly. A token's result
// depends only on its own span and the split grid, so a batch gives every
// token the bits of its one-token call. Addresses are 64-bit.
#include "device_common.h"
#include "kernels.h"

namespace nnchip
{
	namespace
	{
		constexpr int kGenThreads = 256;
		constexpr int kGenChunk = 256; // keys per score chunk (one per thread)
		constexpr int kGenMaxOut = kGenMaxGroupDim / kGenThreads; // outputs per thread

		__device__ __forceinline__ float load_kv(const void* base, size_t i, bool bf16)
		{
			return bf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(base)[i]) : static_cast<const float*>(base)[i];
		}

		// The max (or sum) over the 256 threads of one value per thread, in a
		// fixed order: within each wavefront by xor shuffles, then over the
		// four wavefronts' results in order. Every thread gets the result.
		template <bool MAX>
		__device__ __forceinline__ float block_reduce(float x, float* s_tmp)
		{
#pragma unroll
			for (int off = 32; off > 0; off >>= 1)
			{
				const float y = __shfl_xor(x, off);
				x = MAX ? fmaxf(x, y) : x + y;
			}
			const int w = threadIdx.x >> 6;
			__syncthreads(); // s_tmp is free
			if ((threadIdx.x & 63) == 0) s_tmp[w] = x;
			__syncthreads();
			float r = s_tmp[0];
#pragma unroll
			for (int i = 1; i < kGenThreads / 64; ++i) r = MAX ? fmaxf(r, s_tmp[i]) : r + s_tmp[i];
			return r;
		}

		template <bool BF16>
		__global__ __launch_bounds__(kGenThreads) void decode_generic_kernel(const decode_params p, int head_dim, int group)
		{
			__shared__ float s_q[kGenMaxGroupDim];
			__shared__ float s_w[kGenMaxGroup][kGenChunk];
			__shared__ float s_tmp[kGenThreads / 64];
			const int hd = head_dim, G = group, GD = G * hd;
			const int split = blockIdx.x, kvh = blockIdx.y, tok = blockIdx.z;
			const int tid = threadIdx.x;
			const size_t q_row = static_cast<size_t>(tok) * p.n_head * hd + static_cast<size_t>(kvh) * GD;

			for (int i = tid; i < GD; i += kGenThreads) s_q[i] = p.q[q_row + i] * p.qscale;

			// This split's keys of the token's span.
			int first, last;
			attn_span(p.causal, p.window, p.pos0 + tok, p.n_seq, first, last);
			const int sb = max(first, p.split_base + split * p.split_keys);
			const int se = min(last, p.split_base + (split + 1) * p.split_keys - 1);

			float o[kGenMaxOut];
#pragma unroll
			for (int j = 0; j < kGenMaxOut; ++j) o[j] = 0.0f;
			float m_run[kGenMaxGroup], l_run[kGenMaxGroup];
#pragma unroll
			for (int g = 0; g < kGenMaxGroup; ++g)
			{
				m_run[g] = -INFINITY;
				l_run[g] = 0.0f;
			}
			__syncthreads();

			const size_t kv_stride = static_cast<size_t>(p.kv_dim);
			const size_t head_off = static_cast<size_t>(kvh) * hd;
			for (int c0 = sb; c0 <= se; c0 += kGenChunk)
			{
				const int nk = min(kGenChunk, se - c0 + 1);
				// Scores: thread t, key c0 + t, every head of the group.
				if (tid < nk)
				{
					const size_t row = static_cast<size_t>((c0 + tid) % p.rows) * kv_stride + head_off;
					for (int g = 0; g < G; ++g)
					{
						float s = 0.0f;
						for (int d = 0; d < hd; ++d) s = fmaf(s_q[g * hd + d], load_kv(p.K, row + d, BF16), s);
						s_w[g][tid] = s;
					}
				}
				__syncthreads();
				// Per head: the chunk max, the new running max, the weights and their sum.
				for (int g = 0; g < G; ++g)
				{
					const float mc = block_reduce<true>(tid < nk ? s_w[g][tid] : -INFINITY, s_tmp);
					const float m_new = fmaxf(m_run[g], mc);
					const float m_use = m_new == -INFINITY ? 0.0f : m_new;
					const float alpha = m_run[g] == -INFINITY ? 0.0f : fast_exp2(m_run[g] - m_use);
					float w = 0.0f;
					if (tid < nk)
					{
						w = fast_exp2(s_w[g][tid] - m_use);
						s_w[g][tid] = w;
					}
					const float lc = block_reduce<false>(w, s_tmp);
					l_run[g] = fmaf(l_run[g], alpha, lc);
					m_run[g] = m_new;
					// The thread's outputs of head g: rescaled here, the chunk added below.
#pragma unroll
					for (int j = 0; j < kGenMaxOut; ++j)
					{
						const int idx = tid + kGenThreads * j;
						if (idx < GD && idx / hd == g) o[j] *= alpha;
					}
				}
				__syncthreads(); // every weight is in s_w
#pragma unroll
				for (int j = 0; j < kGenMaxOut; ++j)
				{
					const int idx = tid + kGenThreads * j;
					if (idx >= GD) break;
					const int g = idx / hd, d = idx % hd;
					float acc = o[j];
					for (int t = 0; t < nk; ++t)
						acc = fmaf(s_w[g][t], load_kv(p.V, static_cast<size_t>((c0 + t) % p.rows) * kv_stride + head_off + d, BF16),
						           acc);
					o[j] = acc;
				}
				__syncthreads(); // s_w is free for the next chunk
			}

			// The split's partial, or (one split) o * (1 / l).
			const int PL = hd + 4;
#pragma unroll
			for (int j = 0; j < kGenMaxOut; ++j)
			{
				const int idx = tid + kGenThreads * j;
				if (idx >= GD) break;
				const int g = idx / hd, d = idx % hd;
				if (p.n_split > 1)
				{
					float* gp = p.part + ((static_cast<size_t>(tok) * p.n_kv + kvh) * p.n_split + split) * G * PL +
					            static_cast<size_t>(g) * PL;
					gp[d] = o[j];
					if (d == 0)
					{
						gp[hd] = m_run[g];
						gp[hd + 1] = l_run[g];
					}
				}
				else
				{
					const float inv = l_run[g] > 0.0f ? 1.0f / l_run[g] : 0.0f;
					const size_t oi = q_row + idx;
					p.out[oi] = gated(o[j] * inv, p.gate, oi);
				}
			}
		}

		// The ordered merge of a token's splits for one query head: M = the
		// largest m, o = sum_s o_s 2^(m_s - M), l likewise, in ascending split
		// order; out = o * (1 / l), 0 when l == 0.
		__global__ __launch_bounds__(kGenThreads) void merge_generic_kernel(const decode_params p, int head_dim, int group)
		{
			const int hd = head_dim, G = group, PL = hd + 4;
			const int qh = blockIdx.x, tok = blockIdx.y;
			const int kvh = qh / G, h = qh % G;
			const int ns = p.n_split;
			const float* hp = p.part + ((static_cast<size_t>(tok) * p.n_kv + kvh) * ns * G + h) * PL;
			const size_t sstride = static_cast<size_t>(G) * PL;
			float M = -INFINITY;
			for (int s = 0; s < ns; ++s) M = fmaxf(M, hp[s * sstride + hd]);
			const float m_use = M == -INFINITY ? 0.0f : M;
			for (int d = threadIdx.x; d < hd; d += kGenThreads)
			{
				float r = 0.0f, L = 0.0f;
				for (int s = 0; s < ns; ++s)
				{
					const float* sp = hp + s * sstride;
					const float f = fast_exp2(sp[hd] - m_use);
					r = fmaf(sp[d], f, r);
					L = fmaf(sp[hd + 1], f, L);
				}
				const float inv = L > 0.0f ? 1.0f / L : 0.0f;
				const size_t oi = (static_cast<size_t>(tok) * p.n_head + qh) * hd + d;
				p.out[oi] = gated(r * inv, p.gate, oi);
			}
		}
	}

	bool launch_decode_generic(const decode_params& p, int n_tok, int head_dim, int group, bool bf16, hipStream_t stream)
	{
		if (!generic_shape_ok(head_dim, group)) return false;
		const dim3 grid(p.n_split, p.n_kv, n_tok);
		if (bf16)
			decode_generic_kernel<true><<<grid, kGenThreads, 0, stream>>>(p, head_dim, group);
		else
			decode_generic_kernel<false><<<grid, kGenThreads, 0, stream>>>(p, head_dim, group);
		if (p.n_split > 1) launch_merge_generic(p, n_tok, head_dim, group, stream);
		return true;
	}

	void launch_merge_generic(const decode_params& p, int n_tok, int head_dim, int group, hipStream_t stream)
	{
		merge_generic_kernel<<<dim3(p.n_kv * group, n_tok), kGenThreads, 0, stream>>>(p, head_dim, group);
	}
}
