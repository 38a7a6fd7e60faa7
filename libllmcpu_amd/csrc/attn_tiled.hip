// Tiled attention for the batches the MFMA prefill kernel does not take: F32
// K/V, and head shapes outside mfma_shape (head_dim a multiple of 16 up to
// 512, any group up to 16). nnc runs these through the same attention core
// as every batch (reference src/libnnc/model.cpp:1750-1757); its embedding
// call (model.cpp:2355-2368) is one such batch: the whole input over an F32
// cache, bidirectional.
//
// Rows are (token, query head) pairs of one KV head, token major. Grid:
// (row blocks of 64, KV heads, key splits of the block's keys). A work-group
// of four wavefronts owns 64 rows, 16 per wavefront, and walks its split's
// keys in steps of 16:
// the step's K and V rows are loaded by all 256 threads (F32 as is, BF16
// widened by a 16-bit shift) into LDS, double-buffered, the next step's
// loads in flight in registers while the current one is computed. Every
// product is fp32 on the matrix cores (v_mfma_f32_16x16x4_f32: exact fp32
// products, fp32 sums):
//   S^T = K . Q^T    16 keys x 16 rows, head_dim / 4 MFMAs. Lane l's row is
//                    l % 16; its Q elements sit in registers, element
//                    (l / 16) * (head_dim / 4) + s in MFMA s (any fixed
//                    permutation of d gives the same dot product), so the
//                    K rows are read from LDS 16 bytes at a time;
//   softmax          per row, in fp32 and log2 units (Q pre-scaled by
//                    scale * log2(e)): weights exp2(s - m) against the row's
//                    offset m, raised only when a score passes it by more
//                    than kTileLazy, and their running sum; keys outside the
//                    row's span weigh exactly 0;
//   O^T += V^T . P^T head_dim / 16 tiles of 16 elements x 4 MFMAs of 4 keys;
//                    P^T comes straight from the score registers (key
//                    4 (l / 16) + s in MFMA s), so the row stays in the lane
//                    and the rescale is in-lane.
// A split writes its partial (o, m, l per row, o and l relative to the
// offset m) and a merge kernel combines each row's splits in order; with one
// split per block the kernel writes o * (1 / l) (0 when l == 0, reference
// nn_ops.cpp:492) directly. Splits are relative to the block's first key, so
// only splits that hold keys of the block exist (the windows of a
// bidirectional or sliding layer, the short spans of a causal chunk's first
// tokens), and the partials take n_tok * n_kv * (largest split count) rows.
#include "device_common.h"
#include "kernels.h"

namespace nnchip
{
	namespace
	{
		constexpr int kTileRows = 16; // rows per wavefront
		constexpr int kTileWaves = 4;
		constexpr int kTileBlock = kTileRows * kTileWaves; // rows per work-group
		constexpr int kTileKeys = 16; // keys per step
		constexpr float kTileLazy = 8.0f; // max growth of a row's scores over its offset (log2 units)

		__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4& c)
		{
			return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
		}

		// max / sum of x over the four lanes l % 16 + 16 j (one row's lanes).
		__device__ __forceinline__ float row4_max(float x)
		{
			const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
			x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
			return max_with_other_half(x);
		}

		__device__ __forceinline__ float row4_sum(float x) { return add_with_other_half(add_with_other_row(x)); }

		// Four elements of K or V row `row` at element e (a multiple of 4) of
		// this head, as fp32.
		template <bool BF16>
		__device__ __forceinline__ float4 load4(const void* base, size_t elem)
		{
			if constexpr (BF16)
			{
				const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + elem);
				return make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
			}
			else
				return *reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem);
		}

		// The keys of row block `blk` (its 64 rows' spans together: both ends
		// of a span move forward with the position) and its splits: split z
		// covers keys b_lo + z * split_keys .. + split_keys - 1, relative to
		// the block's first key, so a block has (b_hi - b_lo) / split_keys + 1
		// of them and the grid's z extent is the largest such count.
		__device__ __forceinline__ void tiled_block_keys(const decode_params& p, int G, int blk, int& b_lo, int& b_hi)
		{
			const int n_rows = p.n_tok * G, r0 = blk * kTileBlock, r1 = min(r0 + kTileBlock, n_rows) - 1;
			int unused;
			attn_span(p.causal, p.window, p.pos0 + r0 / G, p.n_seq, b_lo, unused);
			attn_span(p.causal, p.window, p.pos0 + r1 / G, p.n_seq, unused, b_hi);
		}

		__device__ __forceinline__ int tiled_block_splits(int b_lo, int b_hi, int split_keys)
		{
			return b_lo <= b_hi ? (b_hi - b_lo) / split_keys + 1 : 0;
		}

		// Row (t, h)'s partial of its block's split z: [token][KV head][z][group][head_dim + 4]
		// (o, then m and l), z below n_split, the grid's z extent.
		__device__ __forceinline__ float* tiled_partial(const decode_params& p, int G, int hd, int t, int kvh, int z, int h)
		{
			const size_t PL = static_cast<size_t>(hd) + 4;
			return p.part + ((static_cast<size_t>(t) * p.n_kv + kvh) * p.n_split + z) * G * PL + static_cast<size_t>(h) * PL;
		}

		// HD: the head_dim when it is fixed at compile time (the common sizes:
		// no runtime bounds inside the MFMA loops), else 0 and head_dim_arg
		// up to HDMAX.
		template <int HD, int HDMAX, bool BF16>
		__global__ __launch_bounds__(64 * kTileWaves)
		__attribute__((amdgpu_waves_per_eu(HDMAX <= 256 ? 2 : 1))) void tiled_kernel(const decode_params p,
		                                                                              int head_dim_arg, int G)
		{
			const int hd = HD ? HD : head_dim_arg;
			constexpr int PMAX = HDMAX + 4; // LDS row pitch (floats) bound
			constexpr int QV = HDMAX / 4; // Q registers per lane
			constexpr int DT = HDMAX / 16; // 16-element tiles of O^T
			constexpr int LPT = (4 * HDMAX + 255) / 256; // float4 loads per thread per tensor and step
			__shared__ __attribute__((aligned(16))) float s_k[2][kTileKeys * PMAX];
			__shared__ __attribute__((aligned(16))) float s_v[2][kTileKeys * PMAX];

			const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
			const int c = lane >> 4, r16 = lane & 15;
			const int kvh = blockIdx.y, split = blockIdx.z;
			const int pitch = hd + 4, q4 = hd / 4, n_dt = hd / 16, n_f4 = 4 * hd; // float4 slots of a step's K
			const int n_rows = p.n_tok * G;
			const int row0 = blockIdx.x * kTileBlock;
			const int row = row0 + wave * kTileRows + r16;
			const bool row_ok = row < n_rows;
			const int t = row_ok ? row / G : 0, h = row_ok ? row % G : 0;
			const size_t qo = (static_cast<size_t>(t) * p.n_head + static_cast<size_t>(kvh) * G + h) * hd;

			// This split's keys: the row's, and the work-group's (the union over
			// its tokens; both ends of a span move forward with the position).
			int b_lo, b_hi;
			tiled_block_keys(p, G, blockIdx.x, b_lo, b_hi);
			if (split >= tiled_block_splits(b_lo, b_hi, p.split_keys)) return; // the whole work-group: no split here
			const int w_lo = b_lo + split * p.split_keys, w_hi = min(b_hi, w_lo + p.split_keys - 1);
			int first, last;
			attn_span(p.causal, p.window, p.pos0 + t, p.n_seq, first, last);
			const int r_lo = row_ok ? max(first, w_lo) : 1, r_hi = row_ok ? min(last, w_hi) : 0;
			const int n_steps = (w_hi - w_lo) / kTileKeys + 1;

			// Q: element (lane / 16) * (hd / 4) + s in register s, log2 units.
			float q[QV];
#pragma unroll
			for (int s4 = 0; s4 < QV / 4; ++s4)
			{
				float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				if (row_ok && s4 < q4 / 4) v = *reinterpret_cast<const float4*>(p.q + qo + c * q4 + 4 * s4);
				q[4 * s4] = v.x * p.qscale;
				q[4 * s4 + 1] = v.y * p.qscale;
				q[4 * s4 + 2] = v.z * p.qscale;
				q[4 * s4 + 3] = v.w * p.qscale;
			}

			// A step's K and V rows into registers: thread slot i = tid + 256 j
			// is key i / (hd / 4), elements 4 (i % (hd / 4)) .. + 3; keys past
			// the work-group's range are zeros.
			const size_t head_off = static_cast<size_t>(kvh) * hd;
			float4 pk[LPT], pv[LPT];
			auto load_step = [&](int st) __attribute__((always_inline))
			{
				const int k0 = w_lo + st * kTileKeys;
#pragma unroll
				for (int j = 0; j < LPT; ++j)
				{
					const int i = tid + 256 * j;
					const int key = i / q4, e = 4 * (i % q4);
					pk[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
					pv[j] = pk[j];
					if (i < n_f4 && k0 + key <= w_hi)
					{
						const size_t el = static_cast<size_t>((k0 + key) % p.rows) * p.kv_dim + head_off + e;
						pk[j] = load4<BF16>(p.K, el);
						pv[j] = load4<BF16>(p.V, el);
					}
				}
			};
			auto store_step = [&](int buf) __attribute__((always_inline))
			{
#pragma unroll
				for (int j = 0; j < LPT; ++j)
				{
					const int i = tid + 256 * j;
					if (i < n_f4)
					{
						const int off = (i / q4) * pitch + 4 * (i % q4);
						*reinterpret_cast<float4*>(&s_k[buf][off]) = pk[j];
						*reinterpret_cast<float4*>(&s_v[buf][off]) = pv[j];
					}
				}
			};

			f32x4 acc[DT];
#pragma unroll
			for (int d = 0; d < DT; ++d) acc[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
			float m_run = -INFINITY, l_run = 0.0f;

			if (n_steps > 0)
			{
				load_step(0);
				store_step(0);
			}
			__syncthreads();
			for (int st = 0; st < n_steps; ++st)
			{
				const int buf = st & 1;
				if (st + 1 < n_steps) load_step(st + 1);
				const int k0 = w_lo + st * kTileKeys;

				// S^T: lane holds keys k0 + 4 c + i of row r16.
				f32x4 sc = {0.0f, 0.0f, 0.0f, 0.0f};
				const float* kp = &s_k[buf][r16 * pitch + c * q4];
#pragma unroll
				for (int s4 = 0; s4 < QV / 4; ++s4)
				{
					if (s4 < q4 / 4)
					{
						const float4 kv = *reinterpret_cast<const float4*>(kp + 4 * s4);
						sc = mfma_f32(kv.x, q[4 * s4], sc);
						sc = mfma_f32(kv.y, q[4 * s4 + 1], sc);
						sc = mfma_f32(kv.z, q[4 * s4 + 2], sc);
						sc = mfma_f32(kv.w, q[4 * s4 + 3], sc);
					}
				}

				// Online softmax of the row.
				float cmax = -INFINITY;
#pragma unroll
				for (int i = 0; i < 4; ++i)
				{
					const int k = k0 + 4 * c + i;
					sc[i] = (k >= r_lo && k <= r_hi) ? sc[i] : -INFINITY;
					cmax = fmaxf(cmax, sc[i]);
				}
				cmax = row4_max(cmax);
				// The row's offset m is raised (to the step's max) only when a
				// score passes it by more than kTileLazy: weights stay in
				// (0, 2^kTileLazy] and the O rescale is rare (a wavefront-wide
				// branch).
				const bool raise = cmax > m_run + kTileLazy;
				if (__builtin_amdgcn_ballot_w64(raise))
				{
					const float alpha = raise && m_run != -INFINITY ? fast_exp2(m_run - cmax) : 1.0f;
					m_run = raise ? cmax : m_run;
					l_run *= alpha;
#pragma unroll
					for (int d = 0; d < DT; ++d) acc[d] *= alpha;
				}
				const float m_use = m_run == -INFINITY ? 0.0f : m_run;
				float pw[4], ls = 0.0f;
#pragma unroll
				for (int i = 0; i < 4; ++i)
				{
					pw[i] = fast_exp2(sc[i] - m_use);
					ls += pw[i];
				}
				l_run += row4_sum(ls);

				// O^T: tile d holds elements 16 d + 4 c + i of row r16.
				const float* vp = &s_v[buf][(4 * c) * pitch + r16];
#pragma unroll
				for (int d = 0; d < DT; ++d)
				{
					if (d < n_dt)
					{
#pragma unroll
						for (int s = 0; s < 4; ++s) acc[d] = mfma_f32(vp[s * pitch + 16 * d], pw[s], acc[d]);
					}
				}

				if (st + 1 < n_steps) store_step(buf ^ 1);
				__syncthreads();
			}

			if (!row_ok) return;
			if (p.n_split > 1)
			{
				float* gp = tiled_partial(p, G, hd, t, kvh, split, h);
#pragma unroll
				for (int d = 0; d < DT; ++d)
					if (d < n_dt) *reinterpret_cast<f32x4*>(gp + 16 * d + 4 * c) = acc[d];
				if (c == 0) *reinterpret_cast<float2*>(gp + hd) = make_float2(m_run, l_run);
			}
			else
			{
				const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
				for (int d = 0; d < DT; ++d)
				{
					if (d < n_dt)
					{
						const size_t oi = qo + 16 * d + 4 * c;
						float4 o;
						o.x = gated(acc[d][0] * inv, p.gate, oi);
						o.y = gated(acc[d][1] * inv, p.gate, oi + 1);
						o.z = gated(acc[d][2] * inv, p.gate, oi + 2);
						o.w = gated(acc[d][3] * inv, p.gate, oi + 3);
						*reinterpret_cast<float4*>(p.out + oi) = o;
					}
				}
			}
		}

		// The merge of row (t, h)'s splits: those of its block that its own
		// span reaches, in order; M = the largest offset m, o = sum o_z
		// 2^(m_z - M), l likewise; out = o * (1 / l), 0 when l == 0. Four rows
		// per work-group, 64 threads per row, four elements per thread and
		// pass.
		__global__ __launch_bounds__(256) void tiled_merge_kernel(const decode_params p, int hd, int G)
		{
			const int n_rows = p.n_tok * G, r = blockIdx.x * 4 + (threadIdx.x >> 6), kvh = blockIdx.y;
			if (r >= n_rows) return;
			const int lane = threadIdx.x & 63, t = r / G, h = r % G;
			int b_lo, b_hi, first, last;
			tiled_block_keys(p, G, r / kTileBlock, b_lo, b_hi);
			attn_span(p.causal, p.window, p.pos0 + t, p.n_seq, first, last);
			const int z0 = first <= last ? (first - b_lo) / p.split_keys : 0;
			const int z1 = first <= last ? (last - b_lo) / p.split_keys : -1;
			float M = -INFINITY;
			for (int z = z0; z <= z1; ++z) M = fmaxf(M, tiled_partial(p, G, hd, t, kvh, z, h)[hd]);
			const float m_use = M == -INFINITY ? 0.0f : M;
			const size_t oi0 = (static_cast<size_t>(t) * p.n_head + static_cast<size_t>(kvh) * G + h) * hd;
			for (int d = 4 * lane; d < hd; d += 256)
			{
				float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				float L = 0.0f;
				for (int z = z0; z <= z1; ++z)
				{
					const float* gp = tiled_partial(p, G, hd, t, kvh, z, h);
					const float f = fast_exp2(gp[hd] - m_use);
					const float4 v = *reinterpret_cast<const float4*>(gp + d);
					acc.x = fmaf(v.x, f, acc.x);
					acc.y = fmaf(v.y, f, acc.y);
					acc.z = fmaf(v.z, f, acc.z);
					acc.w = fmaf(v.w, f, acc.w);
					L = fmaf(gp[hd + 1], f, L);
				}
				const float inv = L > 0.0f ? 1.0f / L : 0.0f;
				const size_t oi = oi0 + d;
				float4 o;
				o.x = gated(acc.x * inv, p.gate, oi);
				o.y = gated(acc.y * inv, p.gate, oi + 1);
				o.z = gated(acc.z * inv, p.gate, oi + 2);
				o.w = gated(acc.w * inv, p.gate, oi + 3);
				*reinterpret_cast<float4*>(p.out + oi) = o;
			}
		}

		template <int HD, int HDMAX>
		void launch_hd(const decode_params& p, int n_tok, int head_dim, int group, bool bf16, hipStream_t stream)
		{
			const dim3 grid((n_tok * group + kTileBlock - 1) / kTileBlock, p.n_kv, p.n_split);
			if (bf16)
				tiled_kernel<HD, HDMAX, true><<<grid, 64 * kTileWaves, 0, stream>>>(p, head_dim, group);
			else
				tiled_kernel<HD, HDMAX, false><<<grid, 64 * kTileWaves, 0, stream>>>(p, head_dim, group);
		}
	}

	bool launch_tiled(const decode_params& p, int n_tok, int head_dim, int group, bool bf16, hipStream_t stream)
	{
		if (!tiled_shape_ok(head_dim, group)) return false;
		switch (head_dim)
		{
		case 64: launch_hd<64, 64>(p, n_tok, head_dim, group, bf16, stream); break;
		case 80: launch_hd<80, 80>(p, n_tok, head_dim, group, bf16, stream); break;
		case 96: launch_hd<96, 96>(p, n_tok, head_dim, group, bf16, stream); break;
		case 128: launch_hd<128, 128>(p, n_tok, head_dim, group, bf16, stream); break;
		case 256: launch_hd<256, 256>(p, n_tok, head_dim, group, bf16, stream); break;
		case 512: launch_hd<512, 512>(p, n_tok, head_dim, group, bf16, stream); break;
		default:
			if (head_dim <= 128)
				launch_hd<0, 128>(p, n_tok, head_dim, group, bf16, stream);
			else if (head_dim <= 256)
				launch_hd<0, 256>(p, n_tok, head_dim, group, bf16, stream);
			else
				launch_hd<0, 512>(p, n_tok, head_dim, group, bf16, stream);
		}
		if (p.n_split > 1)
			tiled_merge_kernel<<<dim3((n_tok * group + 3) / 4, p.n_kv), 256, 0, stream>>>(p, head_dim, group);
		return true;
	}
}
