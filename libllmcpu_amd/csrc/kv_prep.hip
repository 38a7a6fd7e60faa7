// The step before the attention core, on the device (reference
// src/libnnc/model.cpp:1616-1691): per-head RMSNorm of Q and K (learned gamma)
// and of V (no gamma, Gemma 4), RoPE of Q and K at the token's position, then
// the K and V rows of each token into the layer's cache at row
// (pos0 + t) % rows, BF16 with nnc's round-to-nearest-even (reference
// runtime.h:106-113) or F32. Q is updated in place, ready for the attention
// call; the K/V inputs are left as they are.
//
// A work-group takes 8 head rows of one token, 2 per wavefront, all loaded at
// once (4 rows, one per wavefront, for up to 16 tokens); a head's head_dim
// values are held 64 lanes wide (coalesced loads and stores) and meet through
// the wavefront's LDS row. Every result has the reference's bits:
//   RMSNorm  the sum of squares as the reference's AVX2 loop takes it: eight
//            fp32 fused multiply-add chains over x[l], x[l + 8], ... (lanes
//            0..7, from the LDS row), summed in hsum_ymm's order, the tail in
//            double; the mean, square root and reciprocal in double, rounded
//            once to fp32 (reference nn_ops.cpp:28-36, 558-632); with gamma
//            y = (x * gamma) * scale, the order its -ffast-math build
//            multiplies in.
//   RoPE     cos and sin of each angle from the host (nnc_hip.hip computes them
//            with the host's libm from the reference's fp32 angle), and each
//            pair as fma(c, a, -(s * b)), fma(s, a, c * b), the contraction the
//            reference's build makes (reference nn_ops.cpp:1830-1873).
#include "device_common.h"
#include "kernels.h"

#include <type_traits>

namespace nnchip
{
	namespace
	{
		constexpr int kWaves = 4; // wavefronts per work-group
		constexpr int kMaxHd = 512; // head_dim bound (the reference's RoPE table holds 256 pairs)

		// Head rows per wavefront, loaded together (RPW): 2 for long batches
		// (a Qwen3-4B 512-token layer: 12.2 us at 4, 11.6 at 2, 11.9 at 1), 1 for
		// up to 16 tokens, where a row's exact-order norm chain is the latency
		// and rows side by side in their own wavefronts finish sooner (one
		// Qwen3-4B decode token: 6.9 -> 3.5 us).

		// Work-group (g, t): head rows 4 RPW g .. 4 RPW g + 4 RPW - 1 of token t, where rows
		// 0 .. n_head - 1 are Q heads (updated in place), then n_kv K heads and
		// n_kv V heads (appended to row (pos0 + t) % rows).
		// NJ = head_dim / 64, rounded up: values per lane in a row; FULL: head_dim
		// is exactly 64 NJ (no lane is masked).
		// A full row's NJ consecutive values of one lane, as one wide access
		// (src null: zeros).
		template <int NJ>
		__device__ __forceinline__ void load_row(const float* src, int lane, float* x)
		{
			if (!src)
			{
#pragma unroll
				for (int j = 0; j < NJ; ++j) x[j] = 0.0f;
				return;
			}
			const float* s = src + lane * NJ;
			if constexpr (NJ == 1)
				x[0] = s[0];
			else if constexpr (NJ == 2)
			{
				const float2 v = *reinterpret_cast<const float2*>(s);
				x[0] = v.x;
				x[1] = v.y;
			}
			else
			{
#pragma unroll
				for (int j = 0; j < NJ; j += 4)
				{
					const float4 v = *reinterpret_cast<const float4*>(s + j);
					x[j] = v.x;
					x[j + 1] = v.y;
					x[j + 2] = v.z;
					x[j + 3] = v.w;
				}
			}
		}

		template <int NJ>
		__device__ __forceinline__ void store_row(float* dst, int lane, const float* x)
		{
			float* d = dst + lane * NJ;
			if constexpr (NJ == 1)
				d[0] = x[0];
			else if constexpr (NJ == 2)
				*reinterpret_cast<float2*>(d) = make_float2(x[0], x[1]);
			else
			{
#pragma unroll
				for (int j = 0; j < NJ; j += 4) *reinterpret_cast<float4*>(d + j) = make_float4(x[j], x[j + 1], x[j + 2], x[j + 3]);
			}
		}

		template <int NJ>
		__device__ __forceinline__ void store_row_bf16(uint16_t* dst, int lane, const float* x)
		{
			uint16_t* d = dst + lane * NJ;
			if constexpr (NJ == 1)
				d[0] = static_cast<uint16_t>(f32_to_bf16_bits(x[0]));
			else if constexpr (NJ == 2)
				*reinterpret_cast<uint32_t*>(d) = pack_bf16x2(x[0], x[1]);
			else
			{
#pragma unroll
				for (int j = 0; j < NJ; j += 4)
					*reinterpret_cast<uint2*>(d + j) = make_uint2(pack_bf16x2(x[j], x[j + 1]), pack_bf16x2(x[j + 2], x[j + 3]));
			}
		}

		template <int NJ, bool FULL, int RPW>
		__global__ __launch_bounds__(64 * kWaves) void prep_kernel(const prep_params p)
		{
			constexpr int kRowsPerWave = RPW, kRowsPerGroup = kWaves * RPW;
			__shared__ float s_x[kWaves][kMaxHd];
			const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
			const int t = blockIdx.y;
			const int hd = p.head_dim;
			const int n_hrows = p.n_head + 2 * p.n_kv;
			const size_t q_dim = static_cast<size_t>(p.n_head) * hd, kv_dim = static_cast<size_t>(p.n_kv) * hd;
			// V rows without a norm into a BF16 cache with a copy (f16_blocks_ok):
			// the launch's last column of work-groups writes them with V's fp16
			// copy by whole 16-byte slot sets, from the V inputs (the rows only
			// round to BF16), and the head-row work-groups take Q and K only.
			const bool v_blocks = p.bf16 && p.V16 && !p.v_norm && f16_blocks_ok(p.rows, p.pos0, gridDim.y);
			const int n_rows_here = v_blocks ? p.n_head + p.n_kv : n_hrows;
			if (v_blocks && static_cast<int>(blockIdx.x) == static_cast<int>(gridDim.x) - 1)
			{
				const int n_tok = gridDim.y, kvd = static_cast<int>(kv_dim);
				auto src = [&](int tt, int c) { return f32_to_bf16_bits(p.v[static_cast<size_t>(tt) * kv_dim + c]); };
				const int items = f16_block_items(p.pos0, n_tok, kvd);
				int delta = 0;
				for (int i = t * 64 * kWaves + threadIdx.x; i < items; i += n_tok * 64 * kWaves)
					delta += f16_block_item(static_cast<uint16_t*>(p.V16), static_cast<uint16_t*>(p.V), p.rows, kvd,
					                        p.pos0, n_tok, i, src);
				if (delta != 0) atomicAdd(p.n_bad, delta);
				return;
			}
			const int half = p.n_rot / 2;
			// Element j of this lane in a row: NJ consecutive values per lane for a
			// full row (one wide load or store per row), else strided by 64.
			auto pos = [&](int j) __attribute__((always_inline)) -> int { return FULL ? lane * NJ + j : lane + 64 * j; };

			auto row_src = [&](int hrow, int& kind, int& head) __attribute__((always_inline)) -> const float*
			{
				kind = hrow < p.n_head ? 0 : hrow < p.n_head + p.n_kv ? 1 : 2;
				head = kind == 0 ? hrow : kind == 1 ? hrow - p.n_head : hrow - p.n_head - p.n_kv;
				return kind == 0 ? p.q + t * q_dim + static_cast<size_t>(head) * hd
				       : kind == 1 ? p.k + t * kv_dim + static_cast<size_t>(head) * hd
				                   : p.v + t * kv_dim + static_cast<size_t>(head) * hd;
			};

			// All of this wavefront's rows in flight at once.
			float x[kRowsPerWave][NJ];
#pragma unroll
			for (int r = 0; r < kRowsPerWave; ++r)
			{
				const int hrow = blockIdx.x * kRowsPerGroup + r * kWaves + wave;
				int kind, head;
				const float* src = hrow < n_rows_here ? row_src(hrow, kind, head) : nullptr;
				if constexpr (FULL)
					load_row<NJ>(src, lane, x[r]);
				else
				{
#pragma unroll
					for (int j = 0; j < NJ; ++j)
					{
						const int i = pos(j);
						x[r][j] = (src && i < hd) ? src[i] : 0.0f;
					}
				}
			}

			// This lane's values of the two gammas, with the rows in flight.
			float gq[NJ], gk[NJ];
#pragma unroll
			for (int j = 0; j < NJ; ++j)
			{
				const int i = pos(j);
				const bool in = FULL || i < hd;
				gq[j] = (p.q_gamma && in) ? p.q_gamma[i] : 1.0f;
				gk[j] = (p.k_gamma && in) ? p.k_gamma[i] : 1.0f;
			}

			// cos and sin of the angles of the pairs lane, lane + 64, ... this
			// lane rotates in every row of the token (no barrier: the loads above
			// are in flight).
			constexpr int NP = kPrepMaxPairs / 64;
			float c_tab[NP], s_tab[NP];
			if (half > 0)
			{
				const float2* cs = p.rope_cs + static_cast<size_t>(t) * half;
#pragma unroll
				for (int u = 0; u < NP; ++u)
				{
					const int i = lane + 64 * u;
					const float2 v = i < half ? cs[i] : make_float2(1.0f, 0.0f);
					c_tab[u] = v.x;
					s_tab[u] = v.y;
				}
			}

#pragma unroll
			for (int r = 0; r < kRowsPerWave; ++r)
			{
				const int hrow = blockIdx.x * kRowsPerGroup + r * kWaves + wave;
				if (hrow >= n_rows_here) break; // uniform over the wavefront
				int kind, head;
				(void)row_src(hrow, kind, head);
				float* xr = x[r];

				// RMSNorm: scale = 1 / sqrt(mean of squares + eps) in double
				// (times fp32 1/dim with gamma, divided by dim without, reference
				// nn_ops.cpp:558-632), the sum of squares in the reference's order.
				const float* gamma = kind == 0 ? p.q_gamma : kind == 1 ? p.k_gamma : nullptr;
				const bool norm = kind == 2 ? p.v_norm != 0 : gamma != nullptr;
				if (norm)
				{
					float* xs = s_x[wave];
#pragma unroll
					for (int j = 0; j < NJ; ++j)
					{
						const int i = pos(j);
						if (FULL || i < hd) xs[i] = xr[j];
					}
					wave_sync();
					// Chain l (lane l < 8): fma over x[l], x[l + 8], ... of the
					// full runs of eight, in ascending order.
					const int body = hd & ~7;
					float chain = 0.0f;
					if (lane < 8)
					{
						if constexpr (FULL)
						{
							// (head_dim = 64 NJ: a chain of 8 NJ, its reads all issued first)
#pragma unroll
							for (int k = 0; k < 8 * NJ; ++k) chain = __builtin_fmaf(xs[lane + 8 * k], xs[lane + 8 * k], chain);
						}
						else
							for (int i = lane; i < body; i += 8) chain = __builtin_fmaf(xs[i], xs[i], chain);
					}
					float c8[8];
#pragma unroll
					for (int l = 0; l < 8; ++l) c8[l] = __shfl(chain, l);
					const float hs = __fadd_rn(__fadd_rn(__fadd_rn(c8[0], c8[4]), __fadd_rn(c8[1], c8[5])),
					                           __fadd_rn(__fadd_rn(c8[2], c8[6]), __fadd_rn(c8[3], c8[7])));
					double sum2 = body > 0 ? static_cast<double>(hs) : 0.0;
					for (int i = body; i < hd; ++i)
						sum2 = __dadd_rn(sum2, __dmul_rn(static_cast<double>(xs[i]), static_cast<double>(xs[i])));
					wave_sync(); // the row buffer is free for RoPE
					const double mean = gamma ? __dmul_rn(sum2, static_cast<double>(p.inv_dim))
					                          : __ddiv_rn(sum2, static_cast<double>(hd));
					const float sc = __double2float_rn(__ddiv_rn(1.0, sqrt(__dadd_rn(mean, static_cast<double>(p.eps)))));
#pragma unroll
					for (int j = 0; j < NJ; ++j)
						xr[j] = gamma ? __fmul_rn(__fmul_rn(xr[j], kind == 0 ? gq[j] : gk[j]), sc) : __fmul_rn(xr[j], sc);
				}

				// RoPE on Q and K: NEOX pairs lanes i and i + n_rot/2, NORM lanes
				// 2i and 2i + 1 (reference nn_ops.cpp:1830-1873); lanes past n_rot
				// pass through.
				if (kind != 2 && half > 0)
				{
					float* xs = s_x[wave];
#pragma unroll
					for (int j = 0; j < NJ; ++j)
					{
						const int i = pos(j);
						if (FULL || i < hd) xs[i] = xr[j];
					}
					wave_sync();
					const int stride = p.mode == 0 ? 1 : 2, partner = p.mode == 0 ? half : 1;
#pragma unroll
					for (int u = 0; u < NP; ++u)
					{
						const int i = lane + 64 * u;
						if (i >= half) break;
						const float c = c_tab[u], sn = s_tab[u];
						const int i0 = i * stride, i1 = i0 + partner;
						const float a = xs[i0], b = xs[i1];
						xs[i0] = __builtin_fmaf(c, a, -__fmul_rn(sn, b));
						xs[i1] = __builtin_fmaf(sn, a, __fmul_rn(c, b));
					}
					wave_sync();
#pragma unroll
					for (int j = 0; j < NJ; ++j)
					{
						const int i = pos(j);
						if (FULL || i < hd) xr[j] = xs[i];
					}
					wave_sync(); // the row buffer is free for the next row
				}

				if (kind == 0)
				{
					float* dst = p.q + t * q_dim + static_cast<size_t>(head) * hd;
					if constexpr (FULL)
						store_row<NJ>(dst, lane, xr);
					else
					{
#pragma unroll
						for (int j = 0; j < NJ; ++j)
						{
							const int i = pos(j);
							if (i < hd) dst[i] = xr[j];
						}
					}
					continue;
				}
				const size_t off = static_cast<size_t>((p.pos0 + t) % p.rows) * kv_dim + static_cast<size_t>(head) * hd;
				void* base = kind == 1 ? p.K : p.V;
				if constexpr (FULL)
				{
					if (p.bf16)
						store_row_bf16<NJ>(static_cast<uint16_t*>(base) + off, lane, xr);
					else
						store_row<NJ>(static_cast<float*>(base) + off, lane, xr);
				}
				else
				{
#pragma unroll
					for (int j = 0; j < NJ; ++j)
					{
						const int i = pos(j);
						if (i >= hd) continue;
						if (p.bf16)
							static_cast<uint16_t*>(base)[off + i] = static_cast<uint16_t>(f32_to_bf16_bits(xr[j]));
						else
							static_cast<float*>(base)[off + i] = xr[j];
					}
				}
				if (p.bf16 && p.V16 && kind == 2)
				{
					// V's fp16 copy of the same row (from its BF16 value), in its
					// blocked layout (f16_copy_index).
					uint16_t* sh = static_cast<uint16_t*>(p.V16);
					const int row = (p.pos0 + t) % p.rows;
					int delta = 0;
#pragma unroll
					for (int j = 0; j < NJ; ++j)
					{
						const int i = pos(j);
						if (i < hd)
						{
							const size_t d16 = f16_copy_index(row, head * hd + i, static_cast<int>(kv_dim));
							const uint16_t s16 = bf16_to_f16_bits(f32_to_bf16_bits(xr[j]));
							delta += bad_delta(sh[d16], s16);
							sh[d16] = s16;
						}
					}
					if (delta != 0) atomicAdd(p.n_bad, delta);
				}
			}
		}
	}

	bool launch_prep(const prep_params& p, int n_tok, hipStream_t stream)
	{
		if (p.head_dim <= 0 || p.head_dim > kMaxHd || p.n_rot / 2 > kPrepMaxPairs) return false;
		auto go = [&](auto rpw_tag)
		{
			constexpr int RPW = decltype(rpw_tag)::value;
			const int rows = p.n_head + 2 * p.n_kv;
			// V rows with V's fp16 copy by slot sets: Q and K rows, then one
			// more column of work-groups (the kernel's v_blocks)
			const bool blocks = p.bf16 && p.V16 && !p.v_norm && f16_blocks_ok(p.rows, p.pos0, n_tok);
			const int hrows = blocks ? p.n_head + p.n_kv : rows;
			const dim3 grid((hrows + kWaves * RPW - 1) / (kWaves * RPW) + (blocks ? 1 : 0), n_tok);
			const dim3 block(64 * kWaves);
			switch (p.head_dim)
			{
			case 64: prep_kernel<1, true, RPW><<<grid, block, 0, stream>>>(p); return;
			case 128: prep_kernel<2, true, RPW><<<grid, block, 0, stream>>>(p); return;
			case 256: prep_kernel<4, true, RPW><<<grid, block, 0, stream>>>(p); return;
			case 512: prep_kernel<8, true, RPW><<<grid, block, 0, stream>>>(p); return;
			default: break;
			}
			const int nj = (p.head_dim + 63) / 64;
			if (nj <= 1)
				prep_kernel<1, false, RPW><<<grid, block, 0, stream>>>(p);
			else if (nj <= 2)
				prep_kernel<2, false, RPW><<<grid, block, 0, stream>>>(p);
			else if (nj <= 4)
				prep_kernel<4, false, RPW><<<grid, block, 0, stream>>>(p);
			else
				prep_kernel<8, false, RPW><<<grid, block, 0, stream>>>(p);
		};
		if (n_tok <= 16)
			go(std::integral_constant<int, 1>{});
		else
			go(std::integral_constant<int, 2>{});
		return true;
	}
}
