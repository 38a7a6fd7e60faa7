// The step before the attention core, on the device (reference
// src/libnnc/model.cpp:1616-1691): per-head RMSNorm of Q and K (learned gamma)
// and of V (no gamma, Gemma 4), RoPE of Q and K at the token's position, then
// the K and V rows of each token into the layer's cache at row
// (pos0 + t) % rows, BF16 with nnc's round-to-nearest-even (reference
// runtime.h:106-113) or F32. Q is updated in place, ready for the attention
// call; the K/V inputs are left as they are.
//
// One wavefront per (token, head row): the head's head_dim values are held
// 64 lanes wide (coalesced loads and stores), the RMSNorm sum is a wavefront
// reduction, and RoPE pairs meet through the wavefront's LDS row. The rotation
// angles follow the reference's schedule: the per-pair frequency
// base^(-2i/n_rot) accumulated step by step in fp32 (computed on the host, the
// same sequence of products), times the position, divided by the pair's
// frequency factor when there is one.
#include "device_common.h"
#include "kernels.h"

namespace nnchip
{
	namespace
	{
		constexpr int kWaves = 4; // head rows per work-group
		constexpr int kMaxHd = 512; // head_dim bound (the reference's RoPE table holds 256 pairs)

		__device__ __forceinline__ float wave_sum(float x)
		{
#pragma unroll
			for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
			return x;
		}

		__global__ __launch_bounds__(64 * kWaves) void prep_kernel(const prep_params p)
		{
			__shared__ float s_x[kWaves][kMaxHd];
			const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
			const int hrow = blockIdx.x * kWaves + wave;
			const int t = blockIdx.y;
			if (hrow >= p.n_head + 2 * p.n_kv) return; // whole wavefront; nothing below synchronises the work-group
			const int hd = p.head_dim;
			const size_t q_dim = static_cast<size_t>(p.n_head) * hd, kv_dim = static_cast<size_t>(p.n_kv) * hd;

			// Row kind: 0 = Q head (in place), 1 = K head, 2 = V head.
			const int kind = hrow < p.n_head ? 0 : hrow < p.n_head + p.n_kv ? 1 : 2;
			const int head = kind == 0 ? hrow : kind == 1 ? hrow - p.n_head : hrow - p.n_head - p.n_kv;
			const float* src = kind == 0 ? p.q + t * q_dim + static_cast<size_t>(head) * hd
			                   : kind == 1 ? p.k + t * kv_dim + static_cast<size_t>(head) * hd
			                               : p.v + t * kv_dim + static_cast<size_t>(head) * hd;

			constexpr int NJ = kMaxHd / 64;
			float x[NJ];
#pragma unroll
			for (int j = 0; j < NJ; ++j)
			{
				const int i = lane + 64 * j;
				x[j] = i < hd ? src[i] : 0.0f;
			}

			// RMSNorm: scale = 1 / sqrt(mean of squares + eps), the mean in
			// double as the reference takes it (times fp32 1/dim with gamma,
			// divided by dim without, reference nn_ops.cpp:558-632).
			const float* gamma = kind == 0 ? p.q_gamma : kind == 1 ? p.k_gamma : nullptr;
			const bool norm = kind == 2 ? p.v_norm != 0 : gamma != nullptr;
			if (norm)
			{
				float ss = 0.0f;
#pragma unroll
				for (int j = 0; j < NJ; ++j) ss = fmaf(x[j], x[j], ss);
				const double sum2 = static_cast<double>(wave_sum(ss));
				const double mean = gamma ? sum2 * static_cast<double>(1.0f / static_cast<float>(hd))
				                          : sum2 / static_cast<double>(hd);
				const float r = static_cast<float>(1.0 / sqrt(mean + static_cast<double>(p.eps)));
#pragma unroll
				for (int j = 0; j < NJ; ++j)
				{
					const int i = lane + 64 * j;
					x[j] = x[j] * r;
					if (gamma && i < hd) x[j] *= gamma[i];
				}
			}

			// RoPE on Q and K: NEOX pairs lanes i and i + n_rot/2, NORM lanes 2i
			// and 2i + 1 (reference nn_ops.cpp:1830-1873); lanes past n_rot pass
			// through.
			if (kind != 2 && p.n_rot > 0)
			{
				float* xs = s_x[wave];
#pragma unroll
				for (int j = 0; j < NJ; ++j)
				{
					const int i = lane + 64 * j;
					if (i < hd) xs[i] = x[j];
				}
				wave_sync();
				const int half = p.n_rot / 2;
				const int stride = p.mode == 0 ? 1 : 2, partner = p.mode == 0 ? half : 1;
				const float rpos = static_cast<float>(p.pos0 + t) * p.pos_scale;
				for (int i = lane; i < half; i += 64)
				{
					float th = rpos * p.inv[i];
					if (p.freq_factors) th /= p.freq_factors[i];
					const float c = cosf(th), s = sinf(th);
					const int i0 = i * stride, i1 = i0 + partner;
					const float a = xs[i0], b = xs[i1];
					xs[i0] = c * a - s * b;
					xs[i1] = s * a + c * b;
				}
				wave_sync();
#pragma unroll
				for (int j = 0; j < NJ; ++j)
				{
					const int i = lane + 64 * j;
					if (i < hd) x[j] = xs[i];
				}
			}

			if (kind == 0)
			{
				float* dst = p.q + t * q_dim + static_cast<size_t>(head) * hd;
#pragma unroll
				for (int j = 0; j < NJ; ++j)
				{
					const int i = lane + 64 * j;
					if (i < hd) dst[i] = x[j];
				}
				return;
			}
			const size_t off = static_cast<size_t>((p.pos0 + t) % p.rows) * kv_dim + static_cast<size_t>(head) * hd;
			void* base = kind == 1 ? p.K : p.V;
#pragma unroll
			for (int j = 0; j < NJ; ++j)
			{
				const int i = lane + 64 * j;
				if (i >= hd) continue;
				if (p.bf16)
					static_cast<uint16_t*>(base)[off + i] = static_cast<uint16_t>(f32_to_bf16_bits(x[j]));
				else
					static_cast<float*>(base)[off + i] = x[j];
			}
		}
	}

	bool launch_prep(const prep_params& p, int n_tok, hipStream_t stream)
	{
		if (p.head_dim <= 0 || p.head_dim > kMaxHd || p.n_rot / 2 > kPrepMaxPairs) return false;
		const int rows = p.n_head + 2 * p.n_kv;
		const dim3 grid((rows + kWaves - 1) / kWaves, n_tok);
		prep_kernel<<<grid, 64 * kWaves, 0, stream>>>(p);
		return true;
	}
}
