// Split-K flash-decode for one query token (the n_tok == 1 case of nnc's
// attention core, reference src/libnnc/model.cpp:1731-1749, whose unit of
// work is a (KV head, 256-key block) pair).
//
// Grid: (n_split, n_kv, n_tok). A work-group of 4 wavefronts owns one KV head
// and one absolute-aligned range of split_keys keys of the query's span; each
// wavefront streams chunks of CH keys, the next chunk's K and V loads in
// flight while the current one is computed:
//   scores   S^T[key][head] = K . Q^T on MFMA (v_mfma_f32_16x16x32_bf16): the
//            16 keys of a tile are the M rows, loaded straight from HBM in
//            the A-operand layout (16 contiguous bytes per lane); the group's
//            query heads are the N columns. Q is split into bf16 hi + lo
//            halves, so the product against the exact bf16 K is near-fp32;
//   softmax  per head (column): the chunk max over keys, exp2 of the
//            log2-scaled scores, a running (m, l) with the usual rescale;
//   P.V      BF16 caches (decode_bf16_kernel): O^T = V^T . P^T on MFMA. The
//            chunk's V rows go to the wavefront's LDS tile and come back
//            transposed (ds_read_b64_tr_b16) as the A operand; P^T, split into
//            bf16 hi + lo, is the B operand straight from the score registers
//            (the key order inside a 32-key step is permuted to match).
//            F32 caches (decode_kernel): on the VALU in fp32, each lane owning
//            consecutive elements of one V row and reading the key's weights
//            for all heads of the group from LDS.
// The four wavefront partials merge in LDS; the work-group's partial
// (o, m, l per head) goes to global scratch, and a second small kernel merges
// the splits of each KV head in split order and writes o / l (0 when l == 0,
// reference nn_ops.cpp:492). The order is fixed, so results are the same run
// to run. (A single-kernel "last work-group merges" scheme needs an
// agent-scope release in every work-group, which on this multi-XCD part
// writes back the XCD's L2: measured 1.7x slower at 32k keys.)
#include "device_common.h"
#include "kernels.h"

#include <cstdlib>
#include <type_traits>

namespace nnchip
{
	namespace
	{
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

		// The work-group's result from its wavefronts' partials in s_wpart
		// (o[head_dim], m, l per column, per wavefront), merged in wavefront
		// order. Column c is query head c % G of token tok0 + c / G; the first
		// n_cols columns are filled. With several splits the result is the
		// split's partial; with one it is o * (1 / l), the expression the split
		// merge ends with, so a token gets the same bits either way.
		template <int HD, int G, int C, int W>
		__device__ __forceinline__ void write_wg_result(const decode_params& p, const float (*s_wpart)[C][HD + 2],
		                                                int tok0, int n_cols, int split, int kvh)
		{
			constexpr int PW = HD + 2, kWaves = W, kThreads = 64 * W;
			const int n_kv = gridDim.y;
			const bool single = p.n_split == 1;
			for (int idx = threadIdx.x; idx < n_cols * PW; idx += kThreads)
			{
				const int c = idx / PW, d = idx % PW;
				const int tok = tok0 + c / G, h = c % G;
				float m = -INFINITY;
#pragma unroll
				for (int w = 0; w < kWaves; ++w) m = fmaxf(m, s_wpart[w][c][HD]);
				const float m_use = m == -INFINITY ? 0.0f : m;
				float* gpart = p.part + ((static_cast<size_t>(tok) * n_kv + kvh) * p.n_split + split) * G * PW + h * PW;
				if (d == HD)
				{
					if (!single) gpart[d] = m;
					continue;
				}
				float r = 0.0f;
#pragma unroll
				for (int w = 0; w < kWaves; ++w)
					r = fmaf(s_wpart[w][c][d], fast_exp2(s_wpart[w][c][HD] - m_use), r);
				if (!single)
					gpart[d] = r;
				else if (d < HD)
				{
					float l = 0.0f;
#pragma unroll
					for (int w = 0; w < kWaves; ++w)
						l = fmaf(s_wpart[w][c][HD + 1], fast_exp2(s_wpart[w][c][HD] - m_use), l);
					const float inv = l > 0.0f ? 1.0f / l : 0.0f;
					const size_t oi = (static_cast<size_t>(tok) * p.n_head + kvh * G + h) * HD + d;
					p.out[oi] = gated(r * inv, p.gate, oi);
				}
			}
		}

		// max over the wavefront, on every lane (DPP within 16-lane rows, then
		// the permlane swaps across rows).
		__device__ __forceinline__ float wave_max_dpp(float x)
		{
			x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false)));
			x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false)));
			x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false)));
			x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false)));
			const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
			x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
			return max_with_other_half(x);
		}

		// Merges the n_split partials of one (token, query head) and writes
		// o * (1 / l) (0 when l == 0, reference nn_ops.cpp:492). One wavefront:
		// every split's (m, l) and o slice is loaded before the first use, the
		// maximum comes from DPP and lane swaps, and o and l are summed in
		// ascending split order, one split at a time, with its weight broadcast
		// by v_readlane. A split outside the token's span holds m = -inf, l = 0,
		// o = 0 and adds exact zeros, so a token's result depends only on its own
		// splits, whatever else the launch covered.
		template <int HD, int G>
		__global__ __launch_bounds__(64) void decode_merge_kernel(const decode_params p)
		{
			constexpr int PW = HD + 2, E = HD / 64, KB = 32, MS = kDecodeMaxSplits / 64;
			typedef float fE __attribute__((ext_vector_type(E)));
			const int kvh = blockIdx.x / G, h = blockIdx.x % G, tok = blockIdx.y;
			const int n_kv = gridDim.x / G;
			const int lane = threadIdx.x;
			const int ns = p.n_split;
			const size_t sstride = static_cast<size_t>(G) * PW;
			const float* hp = p.part + ((static_cast<size_t>(tok) * n_kv + kvh) * ns * G + h) * PW; // split s at hp + s * sstride

			float m[MS], l[MS];
#pragma unroll
			for (int j = 0; j < MS; ++j)
			{
				const int s = lane + 64 * j;
				m[j] = s < ns ? hp[s * sstride + HD] : -INFINITY;
				l[j] = s < ns ? hp[s * sstride + HD + 1] : 0.0f;
			}
			fE v[KB];
			auto load_batch = [&](int b0) __attribute__((always_inline))
			{
#pragma unroll
				for (int u = 0; u < KB; ++u)
				{
					const int s = min(b0 + u, ns - 1);
					v[u] = *reinterpret_cast<const fE*>(hp + s * sstride + E * lane);
				}
			};
			load_batch(0);

			float mx = m[0];
#pragma unroll
			for (int j = 1; j < MS; ++j) mx = fmaxf(mx, m[j]);
			mx = wave_max_dpp(mx);
			const float m_use = mx == -INFINITY ? 0.0f : mx;
			float f[MS];
#pragma unroll
			for (int j = 0; j < MS; ++j) f[j] = lane + 64 * j < ns ? fast_exp2(m[j] - m_use) : 0.0f;

			fE acc = fE(0.0f);
			float L = 0.0f;
			for (int b0 = 0;; b0 += KB)
			{
				const int g = b0 >> 6; // uniform; KB divides 64
				float fg = f[0], lg = l[0];
#pragma unroll
				for (int j = 1; j < MS; ++j)
				{
					fg = g == j ? f[j] : fg;
					lg = g == j ? l[j] : lg;
				}
#pragma unroll
				for (int u = 0; u < KB; ++u)
				{
					if (b0 + u < ns) // uniform
					{
						const int src = (b0 & 63) + u;
						const float fw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(fg), src));
						const float lw = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lg), src));
#pragma unroll
						for (int e = 0; e < E; ++e) acc[e] = fmaf(v[u][e], fw, acc[e]);
						L = fmaf(lw, fw, L);
					}
				}
				if (b0 + KB >= ns) break;
				load_batch(b0 + KB);
			}
			const float inv = L > 0.0f ? 1.0f / L : 0.0f;
			const size_t oi = (static_cast<size_t>(tok) * p.n_head + kvh * G + h) * HD + E * lane;
			fE r;
#pragma unroll
			for (int e = 0; e < E; ++e) r[e] = gated(acc[e] * inv, p.gate, oi + e);
			*reinterpret_cast<fE*>(p.out + oi) = r;
		}

		template <int HD, int G, bool BF16, int W>
		__global__ __launch_bounds__(64 * W) void decode_kernel(const decode_params p)
		{
			constexpr int kWaves = W, kThreads = 64 * W;
			using S = decode_shape<HD, BF16>;
			constexpr int CH = S::CH, NT = S::NT, KK = S::KK, VEC = S::VEC, LPK = S::LPK, KPL = S::KPL, NV = S::NV;
			constexpr int PW = HD + 2;

			__shared__ float s_p[kWaves][CH][16]; // weights: [wave][key][head]
			__shared__ float s_alpha[kWaves][16];
			__shared__ float s_wpart[kWaves][G][PW];

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: keeps chunk control flow scalar
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

			float m_run = -INFINITY; // per column (head), log2 units
			float l_run = 0.0f; // this lane's share of the column's sum
			float o[G][VEC];
#pragma unroll
			for (int h = 0; h < G; ++h)
#pragma unroll
				for (int e = 0; e < VEC; ++e) o[h][e] = 0.0f;

			// This wavefront's chunks: CH keys each, every kWaves-th chunk of the
			// split that meets [s0, s1]. Software-pipelined: the V rows of chunk
			// j load during its scores, the K rows of chunk j + 1 during its P.V.
			const int c_first = s0 <= s1 ? (s0 - sbase) / CH : 0;
			const int c_last = s0 <= s1 ? (s1 - sbase) / CH : -1;
			int c_wave = c_first + ((wave - c_first % kWaves) + kWaves) % kWaves;

			uint4 kreg[NT][KK][BF16 ? 1 : 2];
			uint4 vreg[NV];
			auto chunk_bounds = [&](int c, int& cbase, int& clo, int& chi, int& rb) __attribute__((always_inline))
			{
				cbase = sbase + c * CH;
				clo = max(s0, cbase);
				chi = min(s1, cbase + CH - 1);
				rb = clo % p.rows;
			};
			auto load_k = [&](int cbase, int clo, int chi, int rb) __attribute__((always_inline))
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
			};
			auto load_v = [&](int cbase, int clo, int chi, int rb) __attribute__((always_inline))
			{
#pragma unroll
				for (int j = 0; j < NV; ++j)
				{
					const int k = min(max(cbase + j * KPL + lane / LPK, clo), chi);
					const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
					const char* vp = static_cast<const char*>(p.V) +
					                 (row * p.kv_dim + head_off + VEC * (lane % LPK)) * (BF16 ? 2 : 4);
					vreg[j] = *reinterpret_cast<const uint4*>(vp);
				}
			};

			if (c_wave <= c_last)
			{
				int cbase, clo, chi, rb;
				chunk_bounds(c_wave, cbase, clo, chi, rb);
				load_k(cbase, clo, chi, rb);
			}

			// (The first K rows are in flight while Q is prepared.)
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

			for (; c_wave <= c_last; c_wave += kWaves)
			{
				int cbase, clo, chi, rb;
				chunk_bounds(c_wave, cbase, clo, chi, rb);
				load_v(cbase, clo, chi, rb);

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
				if (c_wave + kWaves <= c_last)
				{
					int nb, nlo, nhi, nrb;
					chunk_bounds(c_wave + kWaves, nb, nlo, nhi, nrb);
					load_k(nb, nlo, nhi, nrb);
				}

				// Chunk max per head, masked keys at -inf.
				float m_loc = -INFINITY;
#pragma unroll
				for (int t = 0; t < NT; ++t)
#pragma unroll
					for (int i = 0; i < 4; ++i)
					{
						const int k = cbase + 16 * t + 4 * grp + i;
						const float sc = (k >= clo && k <= chi) ? acc[t][i] : -INFINITY;
						acc[t][i] = sc;
						m_loc = fmaxf(m_loc, sc);
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
				wave_sync();

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
				wave_sync(); // the weights are read before the next chunk overwrites them
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

			write_wg_result<HD, G, G, W>(p, s_wpart, tok, G, split, kvh);
		}

		// Chunk sizes of the BF16 kernel: CH keys per wavefront chunk (a chunk's
		// K and V rows take CH * HD / 128 VGPRs each).
		template <int HD, int CHK>
		struct bf16_shape
		{
			static constexpr int CH = CHK;
			static constexpr int NT = CH / 16; // 16-key MFMA tiles
			static constexpr int NC = CH / 32; // 32-key P.V MFMA steps
			static constexpr int KK = HD / 32;
			static constexpr int DB = HD / 16; // 16-row d blocks of O^T
			static constexpr int LPK = HD / 8; // lanes per V row
			static constexpr int KPL = 64 / LPK; // V rows per load
			static constexpr int NV = CH / KPL; // V loads per chunk
			// LDS pitch of a V row, in bf16: 8 dwords past a multiple of 64 banks,
			// so the four rows one 16-lane group reads with ds_read_b64_tr_b16 sit
			// in disjoint banks (measured: a pitch of head_dim + 8 conflicts).
			static constexpr int VPITCH = HD <= 128 ? 144 : 272;
			static_assert(NC >= 1 && NV >= 1, "unsupported decode shape");
		};

		// Two bf16 halves of one row of O^T's A operand: lane (g, c) of the
		// ds_read_b64_tr_b16 gives V[key0 + 4g + k][d0 + c], k = 0..3, when lane
		// c of each 16-lane group points at V[key0 + 4g + c / 4][d0 + 4 (c % 4)]
		// (the transpose works within 16-lane groups: result element k of lane
		// c comes from lane 4k + c / 4, element c % 4).
		__device__ __forceinline__ u32x2 vt_read(const uint16_t* row_ptr)
		{
			typedef short s16x4 __attribute__((ext_vector_type(4)));
			typedef __attribute__((address_space(3))) s16x4* lds_s16x4;
			const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(row_ptr));
			return __builtin_bit_cast(u32x2, v);
		}

		// BF16 K/V: both products on MFMA.
		//   S^T = K . Q^T     as in decode_kernel (Q split into bf16 hi + lo).
		//   O^T += V^T . P^T  v_mfma_f32_16x16x32_bf16. P^T comes straight from
		//                     the registers that hold S^T: two 16-key tiles give
		//                     a lane the 8 weights it supplies as B operand, keys
		//                     32c + 16h + 4g + k in k-slot 8g + 4h + k. V rows go
		//                     to a per-wavefront LDS tile as loaded, and the A
		//                     operand (V^T) is read back with ds_read_b64_tr_b16
		//                     in that same key order. P is split into bf16 hi + lo,
		//                     so both products are near-fp32 against the exact
		//                     bf16 K and V. O^T's columns are the (token, head)
		//                     pairs, so the online-softmax rescale stays in the
		//                     lane.
		// The 16 MFMA columns hold up to T = 16 / G tokens of G query heads: the
		// tokens of a batch share every K and V load, and each column is masked
		// to its own token's span. A chunk outside a column's span leaves that
		// column's state bit-for-bit unchanged (its weights are exact zeros and
		// its rescale factor exactly 1), so a token gets the same bits alone as
		// in any batch over the same split grid.
		// Loads run one chunk ahead: a chunk's K registers are reissued as soon
		// as its scores are done, its V registers as soon as they are in LDS.
		template <int HD, int G, int W, int CHK, int T>
		__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(1, 1))) void decode_bf16_kernel(
			const decode_params p)
		{
			using S = bf16_shape<HD, CHK>;
			constexpr int CH = S::CH, NT = S::NT, NC = S::NC, KK = S::KK, DB = S::DB, LPK = S::LPK, KPL = S::KPL,
			              NV = S::NV, VPITCH = S::VPITCH;
			constexpr int PW = HD + 2, kWaves = W;
			static_assert(T >= 1 && T * G <= 16, "tokens per work-group");

			__shared__ __attribute__((aligned(16))) uint16_t s_v[W][CH * VPITCH];
			__shared__ float s_wpart[W][T * G][PW];

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: keeps chunk control flow scalar
			const int col = lane & 15;
			const int grp = lane >> 4;
			// A batch's token groups of one (split, KV head) pair go to one XCD
			// in consecutive slots (work-groups are dealt to the XCDs round-robin
			// by linear index), so they stream the same K/V rows through one L2.
			int kvh = blockIdx.y, split = blockIdx.x, zg = blockIdx.z;
			{
				const int nxy = gridDim.x * gridDim.y, nz = gridDim.z;
				const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
				if (nz > 1 && nxy % 8 == 0)
				{
					const int xcd = lin % 8, slot = lin / 8;
					zg = slot % nz;
					const int pair = 8 * (slot / nz) + xcd;
					split = pair % gridDim.x;
					kvh = pair / gridDim.x;
				}
			}
			const int tok0 = zg * T;
			const int n_tt = min(T, p.n_tok - tok0); // tokens of this work-group
			const int tt = col / G; // this lane's column: token tok0 + tt, head col % G

			const int sbase = p.split_base + split * p.split_keys;
			const int send = sbase + p.split_keys - 1;
			// The column's keys in this split (none for a column past the batch),
			// and the work-group's: the union over its tokens, [first of the first
			// token, last of the last] (both ends move forward with the position).
			int first, last;
			attn_span(p.causal, p.window, p.pos0 + tok0 + tt, p.n_seq, first, last);
			const int col_s0 = tt < n_tt ? max(first, sbase) : 1;
			const int col_s1 = tt < n_tt ? min(last, send) : 0;
			int f0, l0, fL, lL;
			attn_span(p.causal, p.window, p.pos0 + tok0, p.n_seq, f0, l0);
			attn_span(p.causal, p.window, p.pos0 + tok0 + n_tt - 1, p.n_seq, fL, lL);
			const int s0 = max(f0, sbase);
			const int s1 = min(lL, send);
			const size_t head_off = static_cast<size_t>(kvh) * HD;
			const uint16_t* Kg = static_cast<const uint16_t*>(p.K) + head_off;
			const uint16_t* Vg = static_cast<const uint16_t*>(p.V) + head_off;
			uint16_t* vt = s_v[wave];

			const int c_first = s0 <= s1 ? (s0 - sbase) / CH : 0;
			const int c_last = s0 <= s1 ? (s1 - sbase) / CH : -1;
			int c_wave = c_first + ((wave - c_first % kWaves) + kWaves) % kWaves;
			const bool has_chunk = c_wave <= c_last; // uniform over the wavefront
			const int n_wchunks = has_chunk ? (c_last - c_wave) / kWaves + 1 : 0;
			const int c_wlast = c_wave + (n_wchunks - 1) * kWaves;

			u32x4 kreg[NT][KK]; // the chunk in flight
			u32x4 vreg[NV];
			auto chunk_bounds = [&](int c, int& cbase, int& clo, int& chi, int& rb) __attribute__((always_inline))
			{
				cbase = sbase + c * CH;
				clo = max(s0, cbase);
				chi = min(s1, cbase + CH - 1);
				rb = clo % p.rows;
			};
			// Loads are never under a branch (a conditional load makes the
			// compiler wait for it, or move the buffer out of registers, where
			// the paths join): a chunk index past the wavefront's last chunk is
			// clamped to it, which re-reads rows that are still in L2.
			auto load_k = [&](int c) __attribute__((always_inline))
			{
				int cbase, clo, chi, rb;
				chunk_bounds(min(c, c_wlast), cbase, clo, chi, rb);
#pragma unroll
				for (int t = 0; t < NT; ++t)
				{
					const int k = min(max(cbase + 16 * t + col, clo), chi);
					const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
					const uint16_t* kp = Kg + row * p.kv_dim + 8 * grp;
#pragma unroll
					for (int kk = 0; kk < KK; ++kk) kreg[t][kk] = *reinterpret_cast<const u32x4*>(kp + 32 * kk);
				}
			};
			// Load j: key j * KPL + lane / LPK, elements 8 * (lane % LPK) .. + 8.
			auto load_v = [&](int c) __attribute__((always_inline))
			{
				int cbase, clo, chi, rb;
				chunk_bounds(min(c, c_wlast), cbase, clo, chi, rb);
#pragma unroll
				for (int j = 0; j < NV; ++j)
				{
					const int k = min(max(cbase + j * KPL + lane / LPK, clo), chi);
					const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
					vreg[j] = *reinterpret_cast<const u32x4*>(Vg + row * p.kv_dim + 8 * (lane % LPK));
				}
			};

			if (has_chunk)
			{
				load_k(c_wave);
				load_v(c_wave);
			}

			// (The first K and V rows are in flight while Q is prepared.) Q^T as
			// the B operand, scaled into log2 units and split into bf16 hi + lo.
			bf16x8 qhi[KK], qlo[KK];
#pragma unroll
			for (int kk = 0; kk < KK; ++kk)
			{
				float x[8];
				if (tt < n_tt)
				{
					const float* qp = p.q + (static_cast<size_t>(tok0 + tt) * p.n_head + kvh * G + col % G) * HD + 32 * kk +
					                  8 * grp;
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

			float m_run = -INFINITY, l_run = 0.0f;
			f32x4 acc_o[DB];
#pragma unroll
			for (int db = 0; db < DB; ++db) acc_o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

			// One chunk from (kreg, vreg); the wavefront's next chunk is loaded
			// into them as soon as they are consumed.
			auto chunk = [&](int cw) __attribute__((always_inline))
			{
				int cbase, clo, chi, rb;
				chunk_bounds(cw, cbase, clo, chi, rb);

				f32x4 sc[NT];
#pragma unroll
				for (int t = 0; t < NT; ++t)
				{
					sc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
					for (int kk = 0; kk < KK; ++kk)
					{
						const bf16x8 a = as_bf16x8(kreg[t][kk]);
						sc[t] = mfma16x16x32(a, qhi[kk], sc[t]);
						sc[t] = mfma16x16x32(a, qlo[kk], sc[t]);
					}
				}
				load_k(cw + kWaves);

				// This chunk's V rows into the wavefront's LDS tile, then the next
				// chunk's V loads into the freed registers.
#pragma unroll
				for (int j = 0; j < NV; ++j)
					*reinterpret_cast<u32x4*>(vt + (j * KPL + lane / LPK) * VPITCH + 8 * (lane % LPK)) = vreg[j];
				load_v(cw + kWaves);

				// Online softmax per head (column).
				float m_loc = -INFINITY;
#pragma unroll
				for (int t = 0; t < NT; ++t)
#pragma unroll
					for (int i = 0; i < 4; ++i)
					{
						const int k = cbase + 16 * t + 4 * grp + i;
						const float v = (k >= col_s0 && k <= col_s1) ? sc[t][i] : -INFINITY;
						sc[t][i] = v;
						m_loc = fmaxf(m_loc, v);
					}
				m_loc = fmaxf(m_loc, __shfl_xor(m_loc, 16));
				m_loc = fmaxf(m_loc, __shfl_xor(m_loc, 32));
				const float m_new = fmaxf(m_run, m_loc);
				const float m_use = m_new == -INFINITY ? 0.0f : m_new;
				const float alpha = fast_exp2(m_run - m_use);
				m_run = m_new;
				float lsum = 0.0f;
				bf16x8 phi[NC], plo[NC];
#pragma unroll
				for (int c = 0; c < NC; ++c)
				{
					float w[8];
#pragma unroll
					for (int i = 0; i < 4; ++i)
					{
						w[i] = fast_exp2(sc[2 * c][i] - m_use);
						w[4 + i] = fast_exp2(sc[2 * c + 1][i] - m_use);
					}
#pragma unroll
					for (int i = 0; i < 8; ++i) lsum += w[i];
					split_bf16x8(w, phi[c], plo[c]);
				}
				l_run = l_run * alpha + lsum;
#pragma unroll
				for (int db = 0; db < DB; ++db) acc_o[db] *= alpha;

				wave_sync();
#pragma unroll
				for (int c = 0; c < NC; ++c)
#pragma unroll
					for (int db = 0; db < DB; ++db)
					{
						const uint16_t* r0 = vt + (32 * c + 4 * grp + (col >> 2)) * VPITCH + 16 * db + 4 * (col & 3);
						const u32x2 lo = vt_read(r0);
						const u32x2 hi = vt_read(r0 + 16 * VPITCH);
						const bf16x8 a = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
						acc_o[db] = mfma16x16x32(a, phi[c], acc_o[db]);
						acc_o[db] = mfma16x16x32(a, plo[c], acc_o[db]);
					}
				wave_sync(); // V is read before the next chunk overwrites it
			};
			for (int i = 0; i < n_wchunks; ++i, c_wave += kWaves) chunk(c_wave);

			// Wavefront partial: each (head, d) of O^T has one owner lane.
			l_run += __shfl_xor(l_run, 16);
			l_run += __shfl_xor(l_run, 32);
			if (tt < n_tt) // col < n_tt * G <= T * G
			{
#pragma unroll
				for (int db = 0; db < DB; ++db)
#pragma unroll
					for (int i = 0; i < 4; ++i) s_wpart[wave][col][16 * db + 4 * grp + i] = acc_o[db][i];
				if (grp == 0)
				{
					s_wpart[wave][col][HD] = m_run;
					s_wpart[wave][col][HD + 1] = l_run;
				}
			}
			__syncthreads();
			write_wg_result<HD, G, T * G, W>(p, s_wpart, tok0, n_tt * G, split, kvh);
		}

		// The BF16 kernel for a session batch: NTL tiles of 16 MFMA columns,
		// 16 * NTL / G tokens per work-group, so a 16-token batch streams each
		// K and V row once. Q (hi and lo) sits in LDS; per chunk the scores of
		// every tile come from the same K registers and the V^T tile is read
		// back once per tile. Each column goes through exactly the operations
		// of decode_bf16_kernel (same products, same order), so a token gets
		// the bits of its one-token call here too.
		template <int HD, int G, int W, int CHK, int NTL>
		__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(1, 1))) void decode_bf16_multi_kernel(
			const decode_params p)
		{
			using S = bf16_shape<HD, CHK>;
			constexpr int CH = S::CH, NT = S::NT, NC = S::NC, KK = S::KK, DB = S::DB, LPK = S::LPK, KPL = S::KPL,
			              NV = S::NV, VPITCH = S::VPITCH;
			constexpr int PW = HD + 2, kWaves = W, T = 16 * NTL / G;
			static_assert(NTL >= 2 && (16 * NTL) % G == 0, "tiles per work-group");

			__shared__ __attribute__((aligned(16))) uint16_t s_v[W][CH * VPITCH];
			__shared__ float s_wpart[W][16][PW];
			__shared__ __attribute__((aligned(16))) u32x4 s_q[NTL][KK][2][64]; // B operands, hi and lo

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
			const int col = lane & 15;
			const int grp = lane >> 4;
			const int kvh = blockIdx.y;
			const int split = blockIdx.x;
			const int tok0 = blockIdx.z * T;
			const int n_tt = min(T, p.n_tok - tok0);

			const int sbase = p.split_base + split * p.split_keys;
			const int send = sbase + p.split_keys - 1;
			int col_s0[NTL], col_s1[NTL];
#pragma unroll
			for (int tl = 0; tl < NTL; ++tl)
			{
				const int tt = (16 * tl + col) / G;
				int first, last;
				attn_span(p.causal, p.window, p.pos0 + tok0 + tt, p.n_seq, first, last);
				col_s0[tl] = tt < n_tt ? max(first, sbase) : 1;
				col_s1[tl] = tt < n_tt ? min(last, send) : 0;
			}
			int f0, l0, fL, lL;
			attn_span(p.causal, p.window, p.pos0 + tok0, p.n_seq, f0, l0);
			attn_span(p.causal, p.window, p.pos0 + tok0 + n_tt - 1, p.n_seq, fL, lL);
			const int s0 = max(f0, sbase);
			const int s1 = min(lL, send);
			const size_t head_off = static_cast<size_t>(kvh) * HD;
			const uint16_t* Kg = static_cast<const uint16_t*>(p.K) + head_off;
			const uint16_t* Vg = static_cast<const uint16_t*>(p.V) + head_off;
			uint16_t* vt = s_v[wave];

			const int c_first = s0 <= s1 ? (s0 - sbase) / CH : 0;
			const int c_last = s0 <= s1 ? (s1 - sbase) / CH : -1;
			int c_wave = c_first + ((wave - c_first % kWaves) + kWaves) % kWaves;
			const bool has_chunk = c_wave <= c_last;
			const int n_wchunks = has_chunk ? (c_last - c_wave) / kWaves + 1 : 0;
			const int c_wlast = c_wave + (n_wchunks - 1) * kWaves;

			u32x4 kreg[NT][KK];
			u32x4 vreg[NV];
			auto chunk_bounds = [&](int c, int& cbase, int& clo, int& chi, int& rb) __attribute__((always_inline))
			{
				cbase = sbase + c * CH;
				clo = max(s0, cbase);
				chi = min(s1, cbase + CH - 1);
				rb = clo % p.rows;
			};
			auto load_k = [&](int c) __attribute__((always_inline))
			{
				int cbase, clo, chi, rb;
				chunk_bounds(min(c, c_wlast), cbase, clo, chi, rb);
#pragma unroll
				for (int t = 0; t < NT; ++t)
				{
					const int k = min(max(cbase + 16 * t + col, clo), chi);
					const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
					const uint16_t* kp = Kg + row * p.kv_dim + 8 * grp;
#pragma unroll
					for (int kk = 0; kk < KK; ++kk) kreg[t][kk] = *reinterpret_cast<const u32x4*>(kp + 32 * kk);
				}
			};
			auto load_v = [&](int c) __attribute__((always_inline))
			{
				int cbase, clo, chi, rb;
				chunk_bounds(min(c, c_wlast), cbase, clo, chi, rb);
#pragma unroll
				for (int j = 0; j < NV; ++j)
				{
					const int k = min(max(cbase + j * KPL + lane / LPK, clo), chi);
					const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
					vreg[j] = *reinterpret_cast<const u32x4*>(Vg + row * p.kv_dim + 8 * (lane % LPK));
				}
			};

			if (has_chunk)
			{
				load_k(c_wave);
				load_v(c_wave);
			}

			// Q^T of every tile into LDS as the B operands, scaled into log2
			// units and split into bf16 hi + lo (entry (tl, kk, l) is lane l's
			// 8 elements 32 kk + 8 (l / 16) .. of column 16 tl + l % 16).
			for (int i = threadIdx.x; i < NTL * KK * 64; i += 64 * W)
			{
				const int l = i & 63, kk = (i >> 6) % KK, tl = (i >> 6) / KK;
				const int gc = 16 * tl + (l & 15), tt = gc / G;
				float x[8];
				if (tt < n_tt)
				{
					const float* qp = p.q + (static_cast<size_t>(tok0 + tt) * p.n_head + kvh * G + gc % G) * HD + 32 * kk +
					                  8 * (l >> 4);
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
				bf16x8 hi, lo;
				split_bf16x8(x, hi, lo);
				s_q[tl][kk][0][l] = __builtin_bit_cast(u32x4, hi);
				s_q[tl][kk][1][l] = __builtin_bit_cast(u32x4, lo);
			}
			__syncthreads();

			float m_run[NTL], l_run[NTL];
			f32x4 acc_o[NTL][DB];
#pragma unroll
			for (int tl = 0; tl < NTL; ++tl)
			{
				m_run[tl] = -INFINITY;
				l_run[tl] = 0.0f;
#pragma unroll
				for (int db = 0; db < DB; ++db) acc_o[tl][db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
			}

			auto chunk = [&](int cw) __attribute__((always_inline))
			{
				int cbase, clo, chi, rb;
				chunk_bounds(cw, cbase, clo, chi, rb);

				f32x4 sc[NTL][NT];
#pragma unroll
				for (int tl = 0; tl < NTL; ++tl)
#pragma unroll
					for (int t = 0; t < NT; ++t) sc[tl][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
				for (int tl = 0; tl < NTL; ++tl)
#pragma unroll
					for (int kk = 0; kk < KK; ++kk)
					{
						const bf16x8 qh = __builtin_bit_cast(bf16x8, s_q[tl][kk][0][lane]);
						const bf16x8 ql = __builtin_bit_cast(bf16x8, s_q[tl][kk][1][lane]);
#pragma unroll
						for (int t = 0; t < NT; ++t)
						{
							const bf16x8 a = as_bf16x8(kreg[t][kk]);
							sc[tl][t] = mfma16x16x32(a, qh, sc[tl][t]);
							sc[tl][t] = mfma16x16x32(a, ql, sc[tl][t]);
						}
					}
				load_k(cw + kWaves);

#pragma unroll
				for (int j = 0; j < NV; ++j)
					*reinterpret_cast<u32x4*>(vt + (j * KPL + lane / LPK) * VPITCH + 8 * (lane % LPK)) = vreg[j];
				load_v(cw + kWaves);
				wave_sync();

#pragma unroll
				for (int tl = 0; tl < NTL; ++tl)
				{
					float m_loc = -INFINITY;
#pragma unroll
					for (int t = 0; t < NT; ++t)
#pragma unroll
						for (int i = 0; i < 4; ++i)
						{
							const int k = cbase + 16 * t + 4 * grp + i;
							const float v = (k >= col_s0[tl] && k <= col_s1[tl]) ? sc[tl][t][i] : -INFINITY;
							sc[tl][t][i] = v;
							m_loc = fmaxf(m_loc, v);
						}
					m_loc = fmaxf(m_loc, __shfl_xor(m_loc, 16));
					m_loc = fmaxf(m_loc, __shfl_xor(m_loc, 32));
					const float m_new = fmaxf(m_run[tl], m_loc);
					const float m_use = m_new == -INFINITY ? 0.0f : m_new;
					const float alpha = fast_exp2(m_run[tl] - m_use);
					m_run[tl] = m_new;
					float lsum = 0.0f;
					bf16x8 phi[NC], plo[NC];
#pragma unroll
					for (int c = 0; c < NC; ++c)
					{
						float w[8];
#pragma unroll
						for (int i = 0; i < 4; ++i)
						{
							w[i] = fast_exp2(sc[tl][2 * c][i] - m_use);
							w[4 + i] = fast_exp2(sc[tl][2 * c + 1][i] - m_use);
						}
#pragma unroll
						for (int i = 0; i < 8; ++i) lsum += w[i];
						split_bf16x8(w, phi[c], plo[c]);
					}
					l_run[tl] = l_run[tl] * alpha + lsum;
#pragma unroll
					for (int db = 0; db < DB; ++db) acc_o[tl][db] *= alpha;
#pragma unroll
					for (int c = 0; c < NC; ++c)
#pragma unroll
						for (int db = 0; db < DB; ++db)
						{
							const uint16_t* r0 = vt + (32 * c + 4 * grp + (col >> 2)) * VPITCH + 16 * db + 4 * (col & 3);
							const u32x2 lo = vt_read(r0);
							const u32x2 hi = vt_read(r0 + 16 * VPITCH);
							const bf16x8 a = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
							acc_o[tl][db] = mfma16x16x32(a, phi[c], acc_o[tl][db]);
							acc_o[tl][db] = mfma16x16x32(a, plo[c], acc_o[tl][db]);
						}
				}
				wave_sync(); // V is read before the next chunk overwrites it
			};
			for (int i = 0; i < n_wchunks; ++i, c_wave += kWaves) chunk(c_wave);

			// One tile at a time through the wavefront merge.
#pragma unroll
			for (int tl = 0; tl < NTL; ++tl)
			{
				float lr = l_run[tl];
				lr += __shfl_xor(lr, 16);
				lr += __shfl_xor(lr, 32);
				const int n_cols = min(16, n_tt * G - 16 * tl); // uniform
				if (col < n_cols)
				{
#pragma unroll
					for (int db = 0; db < DB; ++db)
#pragma unroll
						for (int i = 0; i < 4; ++i) s_wpart[wave][col][16 * db + 4 * grp + i] = acc_o[tl][db][i];
					if (grp == 0)
					{
						s_wpart[wave][col][HD] = m_run[tl];
						s_wpart[wave][col][HD + 1] = lr;
					}
				}
				__syncthreads();
				if (n_cols > 0) write_wg_result<HD, G, 16, W>(p, s_wpart, tok0 + 16 * tl / G, n_cols, split, kvh);
				__syncthreads(); // the partials are read before the next tile overwrites them
			}
		}

		// Keys per wavefront chunk of the BF16 kernel (4 wavefronts, one per
		// SIMD). Measured at 32k keys: 8 wavefronts of 32-key chunks (two per
		// SIMD) run 2% slower.
		constexpr int bf16_chunk(int head_dim) { return head_dim == 256 ? 32 : 64; }

		int bf16_wg_keys(int head_dim) { return 4 * bf16_chunk(head_dim); }

		// NNC_HIP_DECODE_KERNEL=valu runs BF16 caches through the VALU P.V
		// kernel instead of the MFMA one (for comparison).
		bool decode_valu_pv()
		{
			static const bool v = []
			{
				const char* e = std::getenv("NNC_HIP_DECODE_KERNEL");
				return e && e[0] == 'v';
			}();
			return v;
		}

		template <int HD, int G, bool BF16>
		void launch_g(const decode_params& p, int n_kv, int n_tok, int waves, hipStream_t stream)
		{
			const dim3 grid(p.n_split, n_kv, n_tok);
			if (BF16 && !decode_valu_pv())
			{
				// One token: the one-token instance (less LDS for partials);
				// batches: 16 / G tokens per work-group. Both compute a token's
				// column with the same operations.
				constexpr int T = 16 / G, TM = 64 / G; // tokens per work-group: one tile, four tiles
				if (n_tok == 1)
					decode_bf16_kernel<HD, G, 4, bf16_chunk(HD), 1><<<grid, 256, 0, stream>>>(p);
				else
				{
					bool multi = false;
					if constexpr (HD <= 128) // (at head_dim 256 four tiles do not fit the registers)
					{
						if (n_tok > T)
						{
							multi = true;
							decode_bf16_multi_kernel<HD, G, 4, bf16_chunk(HD), 4>
								<<<dim3(p.n_split, n_kv, (n_tok + TM - 1) / TM), 256, 0, stream>>>(p);
						}
					}
					if (!multi)
						decode_bf16_kernel<HD, G, 4, bf16_chunk(HD), T>
							<<<dim3(p.n_split, n_kv, (n_tok + T - 1) / T), 256, 0, stream>>>(p);
				}
			}
			else if (waves == 8)
				decode_kernel<HD, G, BF16, 8><<<grid, 512, 0, stream>>>(p);
			else
				decode_kernel<HD, G, BF16, 4><<<grid, 256, 0, stream>>>(p);
			if (p.n_split > 1) decode_merge_kernel<HD, G><<<dim3(n_kv * G, n_tok), 64, 0, stream>>>(p);
		}

		template <int HD, bool BF16>
		bool launch_hd(const decode_params& p, int n_kv, int n_tok, int group, int waves, hipStream_t stream)
		{
			switch (group)
			{
			case 1: launch_g<HD, 1, BF16>(p, n_kv, n_tok, waves, stream); return true;
			case 2: launch_g<HD, 2, BF16>(p, n_kv, n_tok, waves, stream); return true;
			case 4: launch_g<HD, 4, BF16>(p, n_kv, n_tok, waves, stream); return true;
			case 8: launch_g<HD, 8, BF16>(p, n_kv, n_tok, waves, stream); return true;
			default: return false;
			}
		}

	}

	int decode_waves()
	{
		static const int w = []
		{
			const char* e = std::getenv("NNC_HIP_DECODE_WAVES"); // 4 or 8, for tuning
			return (e && std::atoi(e) == 8) ? 8 : 4;
		}();
		return w;
	}

	int decode_wg_keys(int head_dim, bool bf16)
	{
		switch (head_dim)
		{
		case 64: return (bf16 && !decode_valu_pv()) ? bf16_wg_keys(64) : (bf16 ? decode_shape<64, true>::CH : decode_shape<64, false>::CH) * decode_waves();
		case 128: return (bf16 && !decode_valu_pv()) ? bf16_wg_keys(128) : (bf16 ? decode_shape<128, true>::CH : decode_shape<128, false>::CH) * decode_waves();
		case 256: return (bf16 && !decode_valu_pv()) ? bf16_wg_keys(256) : (bf16 ? decode_shape<256, true>::CH : decode_shape<256, false>::CH) * decode_waves();
		default: return 0;
		}
	}

	bool launch_decode(const decode_params& p, int n_kv, int n_tok, int head_dim, int group, bool bf16,
	                   hipStream_t stream)
	{
		const int w = decode_waves();
		switch (head_dim)
		{
		case 64:
			return bf16 ? launch_hd<64, true>(p, n_kv, n_tok, group, w, stream)
			            : launch_hd<64, false>(p, n_kv, n_tok, group, w, stream);
		case 128:
			return bf16 ? launch_hd<128, true>(p, n_kv, n_tok, group, w, stream)
			            : launch_hd<128, false>(p, n_kv, n_tok, group, w, stream);
		case 256:
			return bf16 ? launch_hd<256, true>(p, n_kv, n_tok, group, w, stream)
			            : launch_hd<256, false>(p, n_kv, n_tok, group, w, stream);
		default: return false;
		}
	}
}
