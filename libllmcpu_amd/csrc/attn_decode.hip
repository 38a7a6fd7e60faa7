// Split-K flash-decode for one query token (the n_tok == 1 case of nnc's
// attention core, reference src/libnnc/model.cpp:1731-1749, whose unit of
// work is a (KV head, 256-key block) pair).
//
// Grid: (n_split, n_kv). A work-group of 4 wavefronts owns one KV head and
// one absolute-aligned range of split_keys keys of the query's span; each
// wavefront streams chunks of CH keys (CH * head_dim * 2 bytes of K and the
// same of V per chunk, all loads issued before any use):
//   scores   S^T[key][head] = K . Q^T on MFMA (v_mfma_f32_16x16x32_bf16): the
//            16 keys of a tile are the M rows, loaded straight from HBM in
//            the A-operand layout (16 contiguous bytes per lane); the group's
//            query heads are the N columns. Q is split into bf16 hi + lo
//            halves, so the product against the exact bf16 K is near-fp32;
//   softmax  per head (column): the chunk max over keys, exp2 of the
//            log2-scaled scores, a running (m, l) with the usual rescale;
//   P.V      on the VALU in fp32: each lane owns 8 consecutive elements of
//            one V row and reads that key's weights for all heads of the
//            group from LDS, so each V element is loaded once for the group.
// The four wavefront partials merge in LDS; the work-group's partial
// (o, m, l per head) goes to global scratch; the last work-group of a KV head
// to arrive (an atomic counter, reset by that work-group) merges all splits
// in split order and writes o / l (0 when l == 0, reference nn_ops.cpp:492).
// The merge order is fixed, so results do not depend on arrival order.
#include "device_common.h"
#include "kernels.h"

namespace nnchip
{
	namespace
	{
		constexpr int kWaves = 4;
		constexpr int kThreads = 64 * kWaves;

		template <int HD, bool BF16>
		struct decode_shape
		{
			static constexpr int VEC = BF16 ? 8 : 4; // elements per 16-byte load
			static constexpr int CH = (BF16 ? 8192 : 4096) / HD; // keys per wave chunk
			static constexpr int NT = CH / 16; // MFMA tiles per chunk
			static constexpr int KK = HD / 32; // MFMA k-steps over head_dim
			static constexpr int LPK = HD / VEC; // lanes per key in the V layout
			static constexpr int KPL = 64 / LPK; // keys per V load
			static constexpr int NV = CH / KPL; // V loads per chunk
			static constexpr int WGK = kWaves * CH; // keys per work-group iteration
			static_assert(NT >= 1 && KK >= 1 && LPK <= 64 && NV >= 1, "unsupported decode shape");
		};

		// Row of key k for k in [lo, hi], with rb = lo % rows. The host
		// guarantees that every span fits the buffer (hi - lo < rows), so the
		// offset from lo wraps at most once.
		__device__ __forceinline__ int ring_row(int k, int lo, int rb, int rows)
		{
			int r = rb + (k - lo);
			return r >= rows ? r - rows : r;
		}

		template <int HD, int G, bool BF16>
		__global__ __launch_bounds__(kThreads) void decode_kernel(const decode_params p)
		{
			using S = decode_shape<HD, BF16>;
			constexpr int CH = S::CH, NT = S::NT, KK = S::KK, VEC = S::VEC, LPK = S::LPK, KPL = S::KPL, NV = S::NV;
			constexpr int PW = HD + 2;

			__shared__ float s_p[kWaves][CH][16]; // weights: [wave][key][head]
			__shared__ float s_alpha[kWaves][16];
			__shared__ float s_wpart[kWaves][G][PW];
			__shared__ float s_w[256 * G]; // final merge: per (split, head) weight
			__shared__ float s_l[G];
			__shared__ int s_last;

			const int lane = threadIdx.x & 63;
			const int wave = threadIdx.x >> 6;
			const int col = lane & 15; // head within the group (MFMA N column)
			const int grp = lane >> 4; // lane group (MFMA K slice / D row quad)
			const int kvh = blockIdx.y;
			const int split = blockIdx.x;
			const int tok = blockIdx.z;
			const int n_kv = gridDim.y;

			int first, last;
			attn_span(p.causal, p.window, p.pos0 + tok, p.n_seq, first, last);
			const int sbase = p.split_base + split * p.split_keys;
			const int s0 = max(first, sbase);
			const int s1 = min(last, sbase + p.split_keys - 1);

			const size_t head_off = static_cast<size_t>(kvh) * HD;
			const float* q = p.q + static_cast<size_t>(tok) * p.n_head * HD;
			float* out = p.out + static_cast<size_t>(tok) * p.n_head * HD;
			const size_t slot = static_cast<size_t>(tok) * n_kv + kvh; // (token, KV head)

			// Q^T as the MFMA B operand: column col = head kvh*G + col, rows
			// 32*kk + 8*grp + j of head_dim; scaled into log2 units, split.
			bf16x8 qhi[KK], qlo[KK];
#pragma unroll
			for (int kk = 0; kk < KK; ++kk)
			{
				float x[8];
				if (col < G)
				{
					const float* qp = q + static_cast<size_t>(kvh * G + col) * HD + 32 * kk + 8 * grp;
					const float4 a = *reinterpret_cast<const float4*>(qp);
					const float4 b = *reinterpret_cast<const float4*>(qp + 4);
					x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
					x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
#pragma unroll
					for (int j = 0; j < 8; ++j) x[j] *= p.qscale;
				}
				else
				{
#pragma unroll
					for (int j = 0; j < 8; ++j) x[j] = 0.0f;
				}
				split_bf16x8(x, qhi[kk], qlo[kk]);
			}

			float m_run = -INFINITY; // per column (head), log2 units
			float l_run = 0.0f; // this lane's share of the column's sum
			float o[G][VEC];
#pragma unroll
			for (int h = 0; h < G; ++h)
#pragma unroll
				for (int e = 0; e < VEC; ++e) o[h][e] = 0.0f;

			const int n_it = p.split_keys / S::WGK;
			for (int it = 0; it < n_it; ++it)
			{
				const int wg_base = sbase + it * S::WGK;
				if (wg_base > s1 || wg_base + S::WGK - 1 < s0) continue; // uniform over the work-group
				const int cbase = wg_base + wave * CH;
				const int clo = max(s0, cbase), chi = min(s1, cbase + CH - 1);
				const bool active = clo <= chi; // uniform over the wave
				const int rb = active ? clo % p.rows : 0;

				uint4 kreg[NT][KK][BF16 ? 1 : 2];
				uint4 vreg[NV];
				if (active)
				{
#pragma unroll
					for (int t = 0; t < NT; ++t)
					{
						const int k = min(max(cbase + 16 * t + col, clo), chi);
						const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
						if constexpr (BF16)
						{
							const uint16_t* kp = static_cast<const uint16_t*>(p.K) + row * p.kv_dim + head_off + 8 * grp;
#pragma unroll
							for (int kk = 0; kk < KK; ++kk) kreg[t][kk][0] = *reinterpret_cast<const uint4*>(kp + 32 * kk);
						}
						else
						{
							const float* kp = static_cast<const float*>(p.K) + row * p.kv_dim + head_off + 8 * grp;
#pragma unroll
							for (int kk = 0; kk < KK; ++kk)
							{
								kreg[t][kk][0] = *reinterpret_cast<const uint4*>(kp + 32 * kk);
								kreg[t][kk][1] = *reinterpret_cast<const uint4*>(kp + 32 * kk + 4);
							}
						}
					}
#pragma unroll
					for (int j = 0; j < NV; ++j)
					{
						const int k = min(max(cbase + j * KPL + lane / LPK, clo), chi);
						const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
						const char* vp = static_cast<const char*>(p.V) +
						                 (row * p.kv_dim + head_off + VEC * (lane % LPK)) * (BF16 ? 2 : 4);
						vreg[j] = *reinterpret_cast<const uint4*>(vp);
					}

					// Scores of the chunk's keys.
					f32x4 acc[NT];
#pragma unroll
					for (int t = 0; t < NT; ++t)
					{
						acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
						for (int kk = 0; kk < KK; ++kk)
						{
							if constexpr (BF16)
							{
								const bf16x8 a = as_bf16x8(kreg[t][kk][0]);
								acc[t] = mfma16x16x32(a, qhi[kk], acc[t]);
								acc[t] = mfma16x16x32(a, qlo[kk], acc[t]);
							}
							else
							{
								float x[8];
								const float* f0 = reinterpret_cast<const float*>(&kreg[t][kk][0]);
								const float* f1 = reinterpret_cast<const float*>(&kreg[t][kk][1]);
#pragma unroll
								for (int j = 0; j < 4; ++j)
								{
									x[j] = f0[j];
									x[4 + j] = f1[j];
								}
								bf16x8 khi, klo;
								split_bf16x8(x, khi, klo);
								acc[t] = mfma16x16x32(khi, qhi[kk], acc[t]);
								acc[t] = mfma16x16x32(khi, qlo[kk], acc[t]);
								acc[t] = mfma16x16x32(klo, qhi[kk], acc[t]);
							}
						}
					}

					// Chunk max per head, masked keys at -inf.
					float m_loc = -INFINITY;
#pragma unroll
					for (int t = 0; t < NT; ++t)
#pragma unroll
						for (int i = 0; i < 4; ++i)
						{
							const int k = cbase + 16 * t + 4 * grp + i;
							const float s = (k >= clo && k <= chi) ? acc[t][i] : -INFINITY;
							acc[t][i] = s;
							m_loc = fmaxf(m_loc, s);
						}
					m_loc = fmaxf(m_loc, __shfl_xor(m_loc, 16));
					m_loc = fmaxf(m_loc, __shfl_xor(m_loc, 32));
					const float m_new = fmaxf(m_run, m_loc);
					const float m_use = m_new == -INFINITY ? 0.0f : m_new;
					const float alpha = fast_exp2(m_run - m_use);
					m_run = m_new;
					float lsum = 0.0f;
#pragma unroll
					for (int t = 0; t < NT; ++t)
#pragma unroll
						for (int i = 0; i < 4; ++i)
						{
							const float w = fast_exp2(acc[t][i] - m_use);
							lsum += w;
							s_p[wave][16 * t + 4 * grp + i][col] = w;
						}
					l_run = l_run * alpha + lsum;
					if (lane < 16) s_alpha[wave][lane] = alpha;
				}
				__syncthreads();
				if (active)
				{
#pragma unroll
					for (int h = 0; h < G; ++h)
					{
						const float a = s_alpha[wave][h];
#pragma unroll
						for (int e = 0; e < VEC; ++e) o[h][e] *= a;
					}
#pragma unroll
					for (int j = 0; j < NV; ++j)
					{
						const int kl = j * KPL + lane / LPK;
						float w[G];
#pragma unroll
						for (int h = 0; h < G; ++h) w[h] = s_p[wave][kl][h];
						float v[VEC];
						if constexpr (BF16)
						{
							const uint32_t* d = reinterpret_cast<const uint32_t*>(&vreg[j]);
#pragma unroll
							for (int u = 0; u < 4; ++u)
							{
								v[2 * u] = bf16_lo(d[u]);
								v[2 * u + 1] = bf16_hi(d[u]);
							}
						}
						else
						{
							const float* f = reinterpret_cast<const float*>(&vreg[j]);
#pragma unroll
							for (int u = 0; u < 4; ++u) v[u] = f[u];
						}
#pragma unroll
						for (int h = 0; h < G; ++h)
#pragma unroll
							for (int e = 0; e < VEC; ++e) o[h][e] = fmaf(w[h], v[e], o[h][e]);
					}
				}
				__syncthreads();
			}

			// Wave partial: sum the key slots of o, the lane groups of l.
#pragma unroll
			for (int off = LPK; off < 64; off *= 2)
#pragma unroll
				for (int h = 0; h < G; ++h)
#pragma unroll
					for (int e = 0; e < VEC; ++e) o[h][e] += __shfl_xor(o[h][e], off);
			l_run += __shfl_xor(l_run, 16);
			l_run += __shfl_xor(l_run, 32);
			if (lane < LPK)
			{
#pragma unroll
				for (int h = 0; h < G; ++h)
#pragma unroll
					for (int e = 0; e < VEC; ++e) s_wpart[wave][h][VEC * lane + e] = o[h][e];
			}
			if (lane < G)
			{
				s_wpart[wave][lane][HD] = m_run;
				s_wpart[wave][lane][HD + 1] = l_run;
			}
			__syncthreads();

			// Work-group partial, waves merged in order.
			float* gpart = p.part + (slot * p.n_split + split) * G * PW;
			for (int idx = threadIdx.x; idx < G * PW; idx += kThreads)
			{
				const int h = idx / PW, d = idx % PW;
				float m = -INFINITY;
#pragma unroll
				for (int w = 0; w < kWaves; ++w) m = fmaxf(m, s_wpart[w][h][HD]);
				const float m_use = m == -INFINITY ? 0.0f : m;
				float r;
				if (d == HD)
					r = m;
				else
				{
					r = 0.0f;
#pragma unroll
					for (int w = 0; w < kWaves; ++w)
					{
						const float f = fast_exp2(s_wpart[w][h][HD] - m_use);
						r = fmaf(s_wpart[w][h][d], f, r);
					}
				}
				gpart[idx] = r;
			}

			// The last work-group of this KV head merges every split.
			__threadfence();
			__syncthreads();
			if (threadIdx.x == 0)
			{
				const unsigned prev = atomicAdd(p.count + slot, 1u);
				s_last = prev == static_cast<unsigned>(p.n_split - 1);
			}
			__syncthreads();
			if (!s_last) return;
			__threadfence();

			const float* kpart = p.part + slot * p.n_split * G * PW;
			for (int idx = threadIdx.x; idx < p.n_split * G; idx += kThreads)
				s_w[idx] = kpart[static_cast<size_t>(idx) * PW + HD];
			__syncthreads();
			if (threadIdx.x < G)
			{
				const int h = threadIdx.x;
				float m = -INFINITY;
				for (int s = 0; s < p.n_split; ++s) m = fmaxf(m, s_w[s * G + h]);
				const float m_use = m == -INFINITY ? 0.0f : m;
				float l = 0.0f;
				for (int s = 0; s < p.n_split; ++s)
				{
					const float f = fast_exp2(s_w[s * G + h] - m_use);
					l = fmaf(kpart[(static_cast<size_t>(s) * G + h) * PW + HD + 1], f, l);
					s_w[s * G + h] = f;
				}
				s_l[h] = l;
			}
			__syncthreads();
			for (int idx = threadIdx.x; idx < G * HD / 4; idx += kThreads)
			{
				const int h = idx / (HD / 4), d = 4 * (idx % (HD / 4));
				float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				for (int s = 0; s < p.n_split; ++s)
				{
					const float f = s_w[s * G + h];
					const float4 v = *reinterpret_cast<const float4*>(kpart + (static_cast<size_t>(s) * G + h) * PW + d);
					acc.x = fmaf(v.x, f, acc.x);
					acc.y = fmaf(v.y, f, acc.y);
					acc.z = fmaf(v.z, f, acc.z);
					acc.w = fmaf(v.w, f, acc.w);
				}
				const float l = s_l[h];
				const float inv = l > 0.0f ? 1.0f / l : 0.0f;
				float* op = out + static_cast<size_t>(kvh * G + h) * HD + d;
				*reinterpret_cast<float4*>(op) = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
			}
			if (threadIdx.x == 0) p.count[slot] = 0u;
		}

		template <int HD, bool BF16>
		bool launch_hd(const decode_params& p, int n_kv, int n_tok, int group, hipStream_t stream)
		{
			const dim3 grid(p.n_split, n_kv, n_tok), block(kThreads);
			switch (group)
			{
			case 1: decode_kernel<HD, 1, BF16><<<grid, block, 0, stream>>>(p); return true;
			case 2: decode_kernel<HD, 2, BF16><<<grid, block, 0, stream>>>(p); return true;
			case 4: decode_kernel<HD, 4, BF16><<<grid, block, 0, stream>>>(p); return true;
			case 8: decode_kernel<HD, 8, BF16><<<grid, block, 0, stream>>>(p); return true;
			default: return false;
			}
		}
	}

	int decode_wg_keys(int head_dim, bool bf16)
	{
		switch (head_dim)
		{
		case 64: return bf16 ? decode_shape<64, true>::WGK : decode_shape<64, false>::WGK;
		case 128: return bf16 ? decode_shape<128, true>::WGK : decode_shape<128, false>::WGK;
		case 256: return bf16 ? decode_shape<256, true>::WGK : decode_shape<256, false>::WGK;
		default: return 0;
		}
	}

	bool launch_decode(const decode_params& p, int n_kv, int n_tok, int head_dim, int group, bool bf16,
	                   hipStream_t stream)
	{
		switch (head_dim)
		{
		case 64:
			return bf16 ? launch_hd<64, true>(p, n_kv, n_tok, group, stream)
			            : launch_hd<64, false>(p, n_kv, n_tok, group, stream);
		case 128:
			return bf16 ? launch_hd<128, true>(p, n_kv, n_tok, group, stream)
			            : launch_hd<128, false>(p, n_kv, n_tok, group, stream);
		case 256:
			return bf16 ? launch_hd<256, true>(p, n_kv, n_tok, group, stream)
			            : launch_hd<256, false>(p, n_kv, n_tok, group, stream);
		default: return false;
		}
	}
}
