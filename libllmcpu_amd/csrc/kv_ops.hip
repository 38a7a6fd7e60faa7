// K/V append with nnc's rounding, the benchmark's synthetic-input generator,
// and a zero fill (used instead of a memset node so the calls stay safe to
// capture in a HIP graph).
#include "device_common.h"
#include "kernels.h"

namespace nnchip
{
	namespace
	{
		// The KV append of reference model.cpp:1668-1691: position pos0 + t goes
		// to row (pos0 + t) % rows; BF16 rounds to nearest even on the bit
		// pattern (reference runtime.h:106-113). Two 16-bit outputs per thread.
		// With a shadow (V16 not null) the fp16 copy of the same V rows is
		// written too, in its blocked layout (f16_copy_index): by whole
		// 16-byte slot sets after the element loop when f16_blocks_ok
		// (f16_block_item, which then writes the V rows as well), else element
		// by element. `n_bad` (the copy's count of kF16Bad elements, values
		// beyond kF16CopyMax) follows the elements replaced and written.
		__global__ void append_bf16_kernel(uint16_t* K, uint16_t* V, const float* k_rows, const float* v_rows,
		                                   int rows, int kv_dim, int pos0, int n_tok, uint16_t* V16,
		                                   int* n_bad)
		{
			const size_t n = static_cast<size_t>(n_tok) * kv_dim;
			const bool blocks = V16 && f16_blocks_ok(rows, pos0, n_tok);
			const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
			const size_t first = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
			int delta = 0;
			for (size_t i = first; i < n; i += stride)
			{
				const int t = static_cast<int>(i / kv_dim);
				const int c = static_cast<int>(i % kv_dim);
				const size_t dst = static_cast<size_t>((pos0 + t) % rows) * kv_dim + c;
				const uint32_t kb = f32_to_bf16_bits(k_rows[i]), vb = f32_to_bf16_bits(v_rows[i]);
				K[dst] = static_cast<uint16_t>(kb);
				if (blocks) continue; // V goes with its copy below
				V[dst] = static_cast<uint16_t>(vb);
				if (V16)
				{
					const size_t d16 = f16_copy_index((pos0 + t) % rows, c, kv_dim);
					const uint16_t v16 = bf16_to_f16_bits(vb);
					delta += bad_delta(V16[d16], v16);
					V16[d16] = v16;
				}
			}
			if (blocks)
			{
				auto src = [&](int t, int c) { return f32_to_bf16_bits(v_rows[static_cast<size_t>(t) * kv_dim + c]); };
				const int items = f16_block_items(pos0, n_tok, kv_dim);
				for (size_t i = first; i < static_cast<size_t>(items); i += stride)
					delta += f16_block_item(V16, V, rows, kv_dim, pos0, n_tok, static_cast<int>(i), src);
			}
			if (delta != 0) atomicAdd(n_bad, delta);
		}

		// The fp16 copy of V rows pos0 .. pos0 + n_tok - 1 (mod rows) of a BF16
		// buffer written by a plain copy; `n_bad` as above.
		__global__ void shadow_rows_kernel(const uint16_t* V, uint16_t* V16,
		                                   int* n_bad, int rows, int kv_dim, int pos0, int n_tok)
		{
			const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
			const size_t first = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
			int delta = 0;
			if (f16_blocks_ok(rows, pos0, n_tok))
			{
				auto src = [&](int t, int c) -> uint32_t { return V[static_cast<size_t>((pos0 + t) % rows) * kv_dim + c]; };
				const int items = f16_block_items(pos0, n_tok, kv_dim);
				for (size_t i = first; i < static_cast<size_t>(items); i += stride)
					delta += f16_block_item(V16, nullptr, rows, kv_dim, pos0, n_tok, static_cast<int>(i), src);
			}
			else
			{
				const size_t n = static_cast<size_t>(n_tok) * kv_dim;
				for (size_t i = first; i < n; i += stride)
				{
					const int t = static_cast<int>(i / kv_dim);
					const int c = static_cast<int>(i % kv_dim);
					const int row = (pos0 + t) % rows;
					const size_t d16 = f16_copy_index(row, c, kv_dim);
					const uint16_t v16 = bf16_to_f16_bits(V[static_cast<size_t>(row) * kv_dim + c]);
					delta += bad_delta(V16[d16], v16);
					V16[d16] = v16;
				}
			}
			if (delta != 0) atomicAdd(n_bad, delta);
		}

		__global__ void append_f32_kernel(float* K, float* V, const float* k_rows, const float* v_rows, int rows,
		                                  int kv_dim, int pos0, int n_tok)
		{
			const size_t n = static_cast<size_t>(n_tok) * kv_dim;
			for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
			     i += static_cast<size_t>(gridDim.x) * blockDim.x)
			{
				const int t = static_cast<int>(i / kv_dim);
				const int c = static_cast<int>(i % kv_dim);
				const size_t dst = static_cast<size_t>((pos0 + t) % rows) * kv_dim + c;
				K[dst] = k_rows[i];
				V[dst] = v_rows[i];
			}
		}

		// splitmix64 (Steele, Lea and Flood, "Fast splittable pseudorandom
		// number generators", 2014): draw i of stream `seed`.
		__device__ __forceinline__ uint64_t splitmix64(uint64_t seed, uint64_t i)
		{
			uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
			z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
			z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
			return z ^ (z >> 31);
		}

		// Box-Muller: element i of the N(0,1) sequence uses draws 2*(i/2) and
		// 2*(i/2) + 1; even i takes the cosine branch, odd i the sine branch.
		__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t i)
		{
			const uint64_t pair = i >> 1;
			const uint64_t a = splitmix64(seed, 2 * pair), b = splitmix64(seed, 2 * pair + 1);
			const double u1 = (static_cast<double>(a >> 11) + 1.0) * 0x1.0p-53;
			const double u2 = static_cast<double>(b >> 11) * 0x1.0p-53;
			const double r = sqrt(-2.0 * log(u1));
			const double th = 6.283185307179586476925 * u2;
			return static_cast<float>((i & 1) ? r * sin(th) : r * cos(th));
		}

		__device__ __forceinline__ void store_elem(void* dst, uint64_t i, float x, bool bf16)
		{
			if (bf16)
				static_cast<uint16_t*>(dst)[i] = static_cast<uint16_t>(f32_to_bf16_bits(x));
			else
				static_cast<float*>(dst)[i] = x;
		}

		__global__ void fill_normal_kernel(void* dst, uint64_t n, uint64_t seed, bool bf16)
		{
			for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < n;
			     i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
				store_elem(dst, i, normal_at(seed, i), bf16);
		}

		// One wavefront per run of norm_dim elements: RMS-normalise (eps 1e-6,
		// sum of squares in fp32), then store.
		__global__ void fill_normal_rms_kernel(void* dst, uint64_t n, uint64_t seed, int norm_dim, bool bf16)
		{
			const uint64_t n_groups = n / norm_dim;
			const int lane = threadIdx.x & 63;
			const uint64_t waves = static_cast<uint64_t>(gridDim.x) * (blockDim.x / 64);
			for (uint64_t g = blockIdx.x * static_cast<uint64_t>(blockDim.x / 64) + (threadIdx.x >> 6); g < n_groups;
			     g += waves)
			{
				const uint64_t base = g * norm_dim;
				float ss = 0.0f;
				for (int j = lane; j < norm_dim; j += 64)
				{
					const float x = normal_at(seed, base + j);
					ss += x * x;
				}
#pragma unroll
				for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
				const float r = 1.0f / sqrtf(ss / static_cast<float>(norm_dim) + 1e-6f);
				for (int j = lane; j < norm_dim; j += 64) store_elem(dst, base + j, normal_at(seed, base + j) * r, bf16);
			}
		}

		// dst[i] = src[i]; src may be pinned host memory (read once, over the
		// bus), dst device memory.
		__global__ void copy_kernel(float* dst, const float* src, size_t n)
		{
			const size_t n4 = n / 4;
			for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n4;
			     i += static_cast<size_t>(gridDim.x) * blockDim.x)
				reinterpret_cast<float4*>(dst)[i] = reinterpret_cast<const float4*>(src)[i];
			if (blockIdx.x == 0 && threadIdx.x < n - 4 * n4) dst[4 * n4 + threadIdx.x] = src[4 * n4 + threadIdx.x];
		}

		__global__ void zero_kernel(float* dst, size_t n)
		{
			for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
			     i += static_cast<size_t>(gridDim.x) * blockDim.x)
				dst[i] = 0.0f;
		}

		unsigned grid_for(size_t n, unsigned block)
		{
			const size_t g = (n + block - 1) / block;
			return static_cast<unsigned>(g < 4096 ? (g > 0 ? g : 1) : 4096);
		}
	}

	bool launch_append_f32(void* K, void* V, const float* k_rows, const float* v_rows, int rows, int kv_dim, int pos0,
	                       int n_tok, bool bf16, hipStream_t stream, void* V16, int* n_bad)
	{
		const size_t n = static_cast<size_t>(n_tok) * kv_dim;
		if (bf16)
			append_bf16_kernel<<<grid_for(n, 256), 256, 0, stream>>>(
				static_cast<uint16_t*>(K), static_cast<uint16_t*>(V), k_rows, v_rows, rows, kv_dim, pos0, n_tok,
				static_cast<uint16_t*>(V16), n_bad);
		else
			append_f32_kernel<<<grid_for(n, 256), 256, 0, stream>>>(static_cast<float*>(K), static_cast<float*>(V), k_rows,
			                                                         v_rows, rows, kv_dim, pos0, n_tok);
		return true;
	}

	bool launch_fill_normal(void* dst, uint64_t n, uint64_t seed, int norm_dim, bool bf16, hipStream_t stream)
	{
		if (norm_dim > 0)
		{
			const uint64_t groups = n / norm_dim;
			fill_normal_rms_kernel<<<grid_for(groups * 64, 256), 256, 0, stream>>>(dst, n, seed, norm_dim, bf16);
		}
		else
			fill_normal_kernel<<<grid_for(n, 256), 256, 0, stream>>>(dst, n, seed, bf16);
		return true;
	}

	bool launch_shadow_rows(const void* V, void* V16, int* n_bad, int rows, int kv_dim, int pos0, int n_tok,
	                        hipStream_t stream)
	{
		const size_t n = static_cast<size_t>(n_tok) * kv_dim;
		shadow_rows_kernel<<<grid_for(n, 256), 256, 0, stream>>>(static_cast<const uint16_t*>(V),
		                                                         static_cast<uint16_t*>(V16), n_bad, rows, kv_dim,
		                                                         pos0, n_tok);
		return true;
	}

	bool launch_copy(float* dst, const float* src, size_t n, hipStream_t stream)
	{
		copy_kernel<<<grid_for((n + 3) / 4, 256), 256, 0, stream>>>(dst, src, n);
		return true;
	}

	bool launch_zero(float* dst, size_t n, hipStream_t stream)
	{
		zero_kernel<<<grid_for(n, 256), 256, 0, stream>>>(dst, n);
		return true;
	}
}
