// Tiled flash attention on CDNA4 MFMA for a batch of query tokens (nnc's
// batch path, reference src/libnnc/model.cpp:1750-1757 and the chunked
// prefill of a long prompt), BF16 K/V.
//
// Precision: the MFMAs run in fp16 with fp32 accumulation. BF16 K/V convert
// to fp16 exactly (8 significant bits fit in 11) for magnitudes up to 65504,
// beyond which they saturate; Q (scaled) and the softmax weights P in [0, 1]
// round to fp16, 8x finer than bf16, which keeps the worst case of a
// first 512-token chunk at Qwen3-4B shape near 1e-3 of nnc's fp32 result.
//
// Rows of the problem are (token, query head) pairs of one KV head, token
// major, so the heads of a GQA group sit in adjacent rows and share every
// K/V tile a work-group stages. Grid: n_kv * n_qtiles work-groups of 4
// wavefronts; a work-group owns 64 * NQ rows, a wavefront 16 * NQ of them.
// The key loop walks 64-key tiles from the first key any row needs to the
// last, staging K ([key][d]) and V^T ([d][key], keys permuted to match the
// register layout of P) in LDS, with the next tile's global loads in flight
// during the current tile's math:
//   S^T = K . Q^T      v_mfma_f32_16x16x32_f16, keys on M, rows on N, so each
//                      lane ends up owning one row's scores: the row max and
//                      sum need only two cross-lane steps;
//   online softmax     in fp32 and log2 units (Q is pre-scaled by
//                      scale * log2 e), masking only tiles that cross a
//                      row's span edge, skipping tiles no row of the
//                      wavefront can see;
//   O^T += V^T . P^T   P stays in registers as the B operand; O^T's columns
//                      are again the lane's own rows, so the rescale is local.
// Masked keys are never read out of bounds: their rows are clamped into the
// tile's valid range and their weights are exactly 0.
#include "device_common.h"
#include "kernels.h"

#include <cstdio>
#include <cstdlib>

namespace nnchip
{
	namespace
	{
		constexpr int kBK = 64; // keys per tile

		// W wavefronts per work-group, each owning 16 * NQ rows.
		template <int HD, int G, int NQ, int W>
		__global__ __launch_bounds__(64 * W) void prefill_kernel(const prefill_params p)
		{
			constexpr int kThreads = 64 * W;
			constexpr int KK = HD / 32; // k-steps of the QK MFMA
			constexpr int DB = HD / 16; // 16-wide d blocks of O^T
			constexpr int KPAD = HD + 8; // LDS row pitch of K, in fp16
			constexpr int VPAD = kBK + 8; // LDS row pitch of V^T, in fp16
			constexpr int ROWS = 16 * NQ * W; // rows per work-group
			constexpr int KCH = kBK * HD / 8 / kThreads; // 16-byte K chunks per thread per tile
			constexpr int VUNITS = (kBK / 4) * (HD / 8); // (4 keys x 8 d) units of V per tile
			constexpr int VUN = (VUNITS + kThreads - 1) / kThreads; // per thread
			static_assert(KCH >= 1 && KCH * kThreads == kBK * HD / 8, "K tile must split evenly over the work-group");

			__shared__ __attribute__((aligned(16))) uint16_t s_k[kBK * KPAD]; // fp16 bits
			__shared__ __attribute__((aligned(16))) uint16_t s_vt[HD * VPAD]; // fp16 bits

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: keeps chunk control flow scalar
			const int col = lane & 15;
			const int grp = lane >> 4;

			// Work-groups of one KV head run on one XCD (blockIdx.x % 8 picks
			// the XCD), so its K/V tiles are shared through that XCD's L2;
			// within a head, the query tiles with the most keys start first.
			int bid = blockIdx.x;
			const int n_wg = gridDim.x;
			if ((n_wg & 7) == 0) bid = (bid & 7) * (n_wg >> 3) + (bid >> 3);
			const int kvh = bid / p.n_qtiles;
			const int qt = p.n_qtiles - 1 - bid % p.n_qtiles;

			const int n_rows = p.n_tok * G;
			const int row0 = qt * ROWS;
			const int wrow0 = row0 + wave * 16 * NQ;
			const size_t q_stride = static_cast<size_t>(p.n_head) * HD;

			// The work-group's key range, and each lane's row spans.
			int kmin, kmax, tmp;
			{
				const int t0 = row0 / G, t1 = min(p.n_tok - 1, (row0 + ROWS - 1) / G);
				attn_span(p.causal, p.window, p.pos0 + t0, p.n_seq, kmin, tmp);
				attn_span(p.causal, p.window, p.pos0 + t1, p.n_seq, tmp, kmax);
			}
			int rfirst[NQ], rlast[NQ];
#pragma unroll
			for (int nb = 0; nb < NQ; ++nb)
			{
				const int r = wrow0 + 16 * nb + col;
				if (r < n_rows)
					attn_span(p.causal, p.window, p.pos0 + r / G, p.n_seq, rfirst[nb], rlast[nb]);
				else
				{
					rfirst[nb] = 1;
					rlast[nb] = 0; // no key
				}
			}
			// The wavefront's own key range (rows are token-major).
			int wfirst, wlast, wfirst_hi, wlast_lo;
			{
				const int ta = min(wrow0 / G, p.n_tok - 1);
				const int tb = min((wrow0 + 16 * NQ - 1) / G, p.n_tok - 1);
				attn_span(p.causal, p.window, p.pos0 + ta, p.n_seq, wfirst, wlast_lo);
				attn_span(p.causal, p.window, p.pos0 + tb, p.n_seq, wfirst_hi, wlast);
			}
			const bool wave_rows = wrow0 < n_rows;

			// Q^T as the B operand, pre-scaled into log2 units, fp16.
			f16x8 qb[NQ][KK];
#pragma unroll
			for (int nb = 0; nb < NQ; ++nb)
			{
				const int r = wrow0 + 16 * nb + col;
				const bool ok = r < n_rows;
				const float* qp = p.q + (ok ? static_cast<size_t>(r / G) * q_stride + static_cast<size_t>(kvh * G + r % G) * HD : 0);
#pragma unroll
				for (int kk = 0; kk < KK; ++kk)
				{
					uint4 w = make_uint4(0u, 0u, 0u, 0u);
					if (ok)
					{
						const float4 a = *reinterpret_cast<const float4*>(qp + 32 * kk + 8 * grp);
						const float4 b = *reinterpret_cast<const float4*>(qp + 32 * kk + 8 * grp + 4);
						const float s = p.qscale;
						w.x = pack_f16x2(a.x * s, a.y * s);
						w.y = pack_f16x2(a.z * s, a.w * s);
						w.z = pack_f16x2(b.x * s, b.y * s);
						w.w = pack_f16x2(b.z * s, b.w * s);
					}
					qb[nb][kk] = as_f16x8(w);
				}
			}

			f32x4 acc_o[DB][NQ];
#pragma unroll
			for (int db = 0; db < DB; ++db)
#pragma unroll
				for (int nb = 0; nb < NQ; ++nb) acc_o[db][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
			float m_run[NQ], l_run[NQ];
#pragma unroll
			for (int nb = 0; nb < NQ; ++nb)
			{
				m_run[nb] = -INFINITY;
				l_run[nb] = 0.0f;
			}

			const uint16_t* Kg = static_cast<const uint16_t*>(p.K) + static_cast<size_t>(kvh) * HD;
			const uint16_t* Vg = static_cast<const uint16_t*>(p.V) + static_cast<size_t>(kvh) * HD;
			const int kb_begin = (kmin / kBK) * kBK;

			uint4 kreg[KCH];
			uint4 vreg[VUN][4];
			auto load_tile = [&](int kb) __attribute__((always_inline))
			{
				// [lo, hi] is never longer than the buffer (checked on the host), so
				// the offset from lo wraps a ring at most once.
				const int lo = max(kb, kmin), hi = min(kb + kBK - 1, kmax);
				const int rb = lo % p.rows;
				auto row_of = [&](int k) __attribute__((always_inline)) -> size_t
				{
					const int kc = min(max(k, lo), hi);
					int r = rb + (kc - lo);
					if (r >= p.rows) r -= p.rows;
					return static_cast<size_t>(r);
				};
#pragma unroll
				for (int u = 0; u < KCH; ++u)
				{
					const int c = threadIdx.x + kThreads * u;
					const int key = c / (HD / 8), d8 = c % (HD / 8);
					kreg[u] = *reinterpret_cast<const uint4*>(Kg + row_of(kb + key) * p.kv_dim + 8 * d8);
				}
#pragma unroll
				for (int u = 0; u < VUN; ++u)
				{
					const int c = threadIdx.x + kThreads * u;
					if (VUNITS % kThreads != 0 && c >= VUNITS) break;
					const int quad = c / (HD / 8), dg = c % (HD / 8);
#pragma unroll
					for (int j = 0; j < 4; ++j)
						vreg[u][j] = *reinterpret_cast<const uint4*>(Vg + row_of(kb + 4 * quad + j) * p.kv_dim + 8 * dg);
				}
			};
			auto store_tile = [&]() __attribute__((always_inline))
			{
#pragma unroll
				for (int u = 0; u < KCH; ++u)
				{
					const int c = threadIdx.x + kThreads * u;
					const int key = c / (HD / 8), d8 = c % (HD / 8);
					const uint4 b = kreg[u];
					uint4 h;
					h.x = pack_f16x2_rtz(bf16_lo(b.x), bf16_hi(b.x));
					h.y = pack_f16x2_rtz(bf16_lo(b.y), bf16_hi(b.y));
					h.z = pack_f16x2_rtz(bf16_lo(b.z), bf16_hi(b.z));
					h.w = pack_f16x2_rtz(bf16_lo(b.w), bf16_hi(b.w));
					*reinterpret_cast<uint4*>(s_k + key * KPAD + 8 * d8) = h;
				}
#pragma unroll
				for (int u = 0; u < VUN; ++u)
				{
					const int c = threadIdx.x + kThreads * u;
					if (VUNITS % kThreads != 0 && c >= VUNITS) break;
					const int quad = c / (HD / 8), dg = c % (HD / 8);
					// Keys 32c + 16h + 4g + j sit at position 32c + 8g + 4h + j.
					const int kq = 4 * quad;
					const int pos = (kq & ~31) + 8 * ((kq >> 2) & 3) + 4 * ((kq >> 4) & 1);
					const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&vreg[u][0]);
					const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&vreg[u][1]);
					const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&vreg[u][2]);
					const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&vreg[u][3]);
#pragma unroll
					for (int e = 0; e < 4; ++e)
					{
						uint2 lo, hi;
						lo.x = pack_f16x2_rtz(bf16_lo(w0[e]), bf16_lo(w1[e]));
						lo.y = pack_f16x2_rtz(bf16_lo(w2[e]), bf16_lo(w3[e]));
						hi.x = pack_f16x2_rtz(bf16_hi(w0[e]), bf16_hi(w1[e]));
						hi.y = pack_f16x2_rtz(bf16_hi(w2[e]), bf16_hi(w3[e]));
						*reinterpret_cast<uint2*>(s_vt + (8 * dg + 2 * e) * VPAD + pos) = lo;
						*reinterpret_cast<uint2*>(s_vt + (8 * dg + 2 * e + 1) * VPAD + pos) = hi;
					}
				}
			};

			if (kb_begin <= kmax) load_tile(kb_begin);
			for (int kb = kb_begin; kb <= kmax; kb += kBK)
			{
				__syncthreads();
				store_tile();
				__syncthreads();
				if (kb + kBK <= kmax) load_tile(kb + kBK);

				// Skip the tile when no row of this wavefront sees any of its keys.
				if (!wave_rows || kb > wlast || kb + kBK - 1 < wfirst) continue;
				const bool edge = kb < wfirst_hi || kb + kBK - 1 > wlast_lo;

				f32x4 s[4][NQ];
#pragma unroll
				for (int mb = 0; mb < 4; ++mb)
#pragma unroll
					for (int nb = 0; nb < NQ; ++nb) s[mb][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
				for (int kk = 0; kk < KK; ++kk)
#pragma unroll
					for (int mb = 0; mb < 4; ++mb)
					{
						const f16x8 a = as_f16x8(*reinterpret_cast<const uint4*>(s_k + (16 * mb + col) * KPAD + 32 * kk + 8 * grp));
#pragma unroll
						for (int nb = 0; nb < NQ; ++nb) s[mb][nb] = mfma16x16x32(a, qb[nb][kk], s[mb][nb]);
					}

				if (edge)
				{
#pragma unroll
					for (int mb = 0; mb < 4; ++mb)
#pragma unroll
						for (int i = 0; i < 4; ++i)
						{
							const int k = kb + 16 * mb + 4 * grp + i;
#pragma unroll
							for (int nb = 0; nb < NQ; ++nb)
								if (k < rfirst[nb] || k > rlast[nb]) s[mb][nb][i] = -INFINITY;
						}
				}

				f16x8 pb[2][NQ];
#pragma unroll
				for (int nb = 0; nb < NQ; ++nb)
				{
					float mt = -INFINITY;
#pragma unroll
					for (int mb = 0; mb < 4; ++mb)
#pragma unroll
						for (int i = 0; i < 4; ++i) mt = fmaxf(mt, s[mb][nb][i]);
					mt = fmaxf(mt, __shfl_xor(mt, 16));
					mt = fmaxf(mt, __shfl_xor(mt, 32));
					const float m_new = fmaxf(m_run[nb], mt);
					const float m_use = m_new == -INFINITY ? 0.0f : m_new;
					const float alpha = fast_exp2(m_run[nb] - m_use);
					m_run[nb] = m_new;
					float pw[4][4];
					float lsum = 0.0f;
#pragma unroll
					for (int mb = 0; mb < 4; ++mb)
#pragma unroll
						for (int i = 0; i < 4; ++i)
						{
							pw[mb][i] = fast_exp2(s[mb][nb][i] - m_use);
							lsum += pw[mb][i];
						}
					l_run[nb] = l_run[nb] * alpha + lsum;
#pragma unroll
					for (int db = 0; db < DB; ++db) acc_o[db][nb] *= alpha;
#pragma unroll
					for (int c = 0; c < 2; ++c)
					{
						uint4 w;
						w.x = pack_f16x2(pw[2 * c][0], pw[2 * c][1]);
						w.y = pack_f16x2(pw[2 * c][2], pw[2 * c][3]);
						w.z = pack_f16x2(pw[2 * c + 1][0], pw[2 * c + 1][1]);
						w.w = pack_f16x2(pw[2 * c + 1][2], pw[2 * c + 1][3]);
						pb[c][nb] = as_f16x8(w);
					}
				}

#pragma unroll
				for (int c = 0; c < 2; ++c)
#pragma unroll
					for (int db = 0; db < DB; ++db)
					{
						const f16x8 a = as_f16x8(*reinterpret_cast<const uint4*>(s_vt + (16 * db + col) * VPAD + 32 * c + 8 * grp));
#pragma unroll
						for (int nb = 0; nb < NQ; ++nb) acc_o[db][nb] = mfma16x16x32(a, pb[c][nb], acc_o[db][nb]);
					}
			}

			// o / l per row (0 when l == 0, reference nn_ops.cpp:492).
#pragma unroll
			for (int nb = 0; nb < NQ; ++nb)
			{
				float l = l_run[nb];
				l += __shfl_xor(l, 16);
				l += __shfl_xor(l, 32);
				const int r = wrow0 + 16 * nb + col;
				if (r >= n_rows) continue;
				const float inv = l > 0.0f ? 1.0f / l : 0.0f;
				float* op = p.out + static_cast<size_t>(r / G) * q_stride + static_cast<size_t>(kvh * G + r % G) * HD + 4 * grp;
#pragma unroll
				for (int db = 0; db < DB; ++db)
				{
					const f32x4 v = acc_o[db][nb];
					*reinterpret_cast<float4*>(op + 16 * db) = make_float4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
				}
			}
		}

		template <int HD, int NQ, int W>
		bool launch_g(const prefill_params& p, int group, hipStream_t stream)
		{
			const dim3 grid(p.n_qtiles * p.n_kv), block(64 * W);
			switch (group)
			{
			case 1: prefill_kernel<HD, 1, NQ, W><<<grid, block, 0, stream>>>(p); return true;
			case 2: prefill_kernel<HD, 2, NQ, W><<<grid, block, 0, stream>>>(p); return true;
			case 4: prefill_kernel<HD, 4, NQ, W><<<grid, block, 0, stream>>>(p); return true;
			case 8: prefill_kernel<HD, 8, NQ, W><<<grid, block, 0, stream>>>(p); return true;
			default: return false;
			}
		}

		// Tile shape (wavefronts per work-group, 16-row blocks per wavefront):
		// NNC_HIP_PREFILL_TILE="W,NQ" overrides the default, for tuning.
		void tile_shape(int head_dim, int& w, int& nq)
		{
			w = 4;
			nq = head_dim == 256 ? 1 : 2;
			if (const char* e = std::getenv("NNC_HIP_PREFILL_TILE"))
			{
				int a = 0, b = 0;
				if (std::sscanf(e, "%d,%d", &a, &b) == 2 && (a == 2 || a == 4) && (b == 1 || b == 2)) w = a, nq = b;
			}
		}
	}

	bool launch_prefill(prefill_params p, int head_dim, int group, bool bf16, hipStream_t stream)
	{
		if (!bf16) return false;
		int w, nq;
		tile_shape(head_dim, w, nq);
		const int rows = 16 * nq * w;
		p.n_qtiles = (p.n_tok * group + rows - 1) / rows;
		switch (head_dim * 100 + w * 10 + nq)
		{
		case 6421: return launch_g<64, 1, 2>(p, group, stream);
		case 6422: return launch_g<64, 2, 2>(p, group, stream);
		case 6441: return launch_g<64, 1, 4>(p, group, stream);
		case 6442: return launch_g<64, 2, 4>(p, group, stream);
		case 12821: return launch_g<128, 1, 2>(p, group, stream);
		case 12822: return launch_g<128, 2, 2>(p, group, stream);
		case 12841: return launch_g<128, 1, 4>(p, group, stream);
		case 12842: return launch_g<128, 2, 4>(p, group, stream);
		case 25621: return launch_g<256, 1, 2>(p, group, stream);
		case 25641: return launch_g<256, 1, 4>(p, group, stream);
		default: return false;
		}
	}
}
