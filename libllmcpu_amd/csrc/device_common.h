// Device-side helpers shared by the attention kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nnchip
{
	// MFMA operand and accumulator types. v_mfma_f32_16x16x32_bf16 takes
	// 8 bf16 of A and 8 of B per lane and accumulates 4 fp32 per lane:
	//   A: lane l holds A[l % 16][8 * (l / 16) + j], j = 0..7   (M x K = 16 x 32)
	//   B: lane l holds B[8 * (l / 16) + j][l % 16]              (K x N = 32 x 16)
	//   D: lane l holds D[4 * (l / 16) + i][l % 16], i = 0..3    (M x N = 16 x 16)
	// v_mfma_f32_16x16x32_f16 has the same operand layout.
	typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
	typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
	typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
	typedef float f32x4 __attribute__((ext_vector_type(4)));
	// 16 bytes as a native vector: register buffers of this type stay in
	// registers (arrays of HIP's uint4 struct can end up in scratch or LDS).
	typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
	typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

	__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c)
	{
		return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
	}

	__device__ __forceinline__ f32x4 mfma16x16x32(const f16x8& a, const f16x8& b, const f32x4& c)
	{
		return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
	}

	// v_mfma_f32_32x32x16_{bf16,f16}: 8 elements of A and of B per lane, 16
	// fp32 accumulators per lane (measured on gfx950: one wavefront keeps these
	// at ~97% of the matrix peak, where 16x16x32 needs two):
	//   A: lane l holds A[l % 32][8 * (l / 32) + j], j = 0..7   (M x K = 32 x 16)
	//   B: lane l holds B[8 * (l / 32) + j][l % 32]              (K x N = 16 x 32)
	//   D: lane l holds D[8 * (i / 4) + 4 * (l / 32) + i % 4][l % 32], i = 0..15
	typedef float f32x16 __attribute__((ext_vector_type(16)));

	__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c)
	{
		return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
	}

	__device__ __forceinline__ f32x16 mfma32x32x16(const f16x8& a, const f16x8& b, const f32x16& c)
	{
		return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
	}

	// max(x[l], x[l ^ 32]) on every lane, without LDS: v_permlane32_swap
	// exchanges one half-wavefront of its two operands, so the two results
	// hold each lane's value and its partner's (in either order).
	__device__ __forceinline__ float max_with_other_half(float x)
	{
		const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
		return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
	}

	__device__ __forceinline__ float add_with_other_half(float x)
	{
		const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
		return __uint_as_float(r[0]) + __uint_as_float(r[1]);
	}

	// x[l] + x[l ^ 16] on every lane (v_permlane16_swap exchanges the odd
	// 16-lane rows of one operand with the even rows of the other).
	__device__ __forceinline__ float add_with_other_row(float x)
	{
		const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
		return __uint_as_float(r[0]) + __uint_as_float(r[1]);
	}

	// The sum of x over the wavefront, on every lane, without LDS: within each
	// 16-lane row by DPP (quad permutations [1,0,3,2] and [2,3,0,1], then the
	// half-row and row mirrors), then across rows with the permlane swaps.
	__device__ __forceinline__ float wave_sum_dpp(float x)
	{
		x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false)); // lane ^ 1
		x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false)); // lane ^ 2
		x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false)); // half-row mirror
		x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false)); // row mirror
		x = add_with_other_row(x);
		return add_with_other_half(x);
	}

	// 16 bytes with the non-temporal hint (global_load_dwordx4 ... nt): for
	// K/V rows that one call reads once. Measured on a 134 MB per-head-slice
	// stream: 22.4 us with the hint, 25.2 us without.
	__device__ __forceinline__ u32x4 load_stream(const void* p)
	{
		return __builtin_nontemporal_load(static_cast<const u32x4*>(p));
	}

	__device__ __forceinline__ f16x8 as_f16x8(const uint4& v) { return __builtin_bit_cast(f16x8, v); }
	__device__ __forceinline__ f16x8 as_f16x8(const u32x4& v) { return __builtin_bit_cast(f16x8, v); }

	// Two fp32 -> packed fp16, rounded to nearest even.
	__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi)
	{
		const f16x2 h = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
		return __builtin_bit_cast(uint32_t, h);
	}

	// nnc's BF16 contract (reference runtime.h:97-113): widen by a 16-bit
	// shift, narrow with round-to-nearest-even on the bit pattern.
	__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

	__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f)
	{
		const uint32_t u = __float_as_uint(f);
		return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
	}

	// The two bf16 halves of one dword as fp32.
	__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
	__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

	__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
	{
		return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
	}

	__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8, v); }
	__device__ __forceinline__ bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

	// Two fp32 -> packed bf16, rounded to nearest even (v_cvt_pk_bf16_f32).
	__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi)
	{
		typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
		const bf16x2 h = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
		return __builtin_bit_cast(uint32_t, h);
	}

	// Splits 8 fp32 values into bf16 hi + lo parts with x ~= hi + lo to about
	// 16 significant bits, so two bf16 MFMAs give a near-fp32 product against
	// an exact bf16 operand.
	__device__ __forceinline__ void split_bf16x8(const float* x, bf16x8& hi, bf16x8& lo)
	{
		u32x4 h, l;
#pragma unroll
		for (int j = 0; j < 4; ++j)
		{
			const float a = x[2 * j], b = x[2 * j + 1];
			const uint32_t hw = cvt_pk_bf16(a, b);
			h[j] = hw;
			l[j] = cvt_pk_bf16(a - bf16_lo(hw), b - bf16_hi(hw));
		}
		hi = as_bf16x8(h);
		lo = as_bf16x8(l);
	}

	// The same split of 4 values (the bits split_bf16x8 gives them), as two
	// packed dwords per half.
	__device__ __forceinline__ void split_bf16x4(const float4& x, u32x2& hi, u32x2& lo)
	{
		const uint32_t h0 = cvt_pk_bf16(x.x, x.y), h1 = cvt_pk_bf16(x.z, x.w);
		hi = u32x2{h0, h1};
		lo = u32x2{cvt_pk_bf16(x.x - bf16_lo(h0), x.y - bf16_hi(h0)), cvt_pk_bf16(x.z - bf16_lo(h1), x.w - bf16_hi(h1))};
	}

	// Orders one wavefront's LDS writes before its own later reads of other
	// lanes' values (LDS executes a wavefront's operations in order; this
	// keeps the compiler from moving them).
	__device__ __forceinline__ void wave_sync()
	{
		__builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
		__builtin_amdgcn_wave_barrier();
		__builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
	}

	__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

	// A float4 store with the non-temporal hint (one global_store_dwordx4 ...
	// nt): for results nothing in the same kernel reads again. A prefill
	// launch's 8 MB of output otherwise stays dirty in L2 until the end of the
	// kernel writes it back (Qwen3-4B prefill 9.70 -> 9.57 ms per step, Gemma-3-4B
	// 25.81 -> 25.21, one process, alternating libraries).
	__device__ __forceinline__ void store_stream(float* dst, float4 v)
	{
		__builtin_nontemporal_store(v.x, dst);
		__builtin_nontemporal_store(v.y, dst + 1);
		__builtin_nontemporal_store(v.z, dst + 2);
		__builtin_nontemporal_store(v.w, dst + 3);
	}

	// The fp16 copy of a BF16 V element kept for the prefill kernel (RNE;
	// exact for every bf16 from 2^-14 up to fp16's range, within 2^-25 below).
	// The prefill kernel multiplies it by P rounded to fp16 (relative error at
	// most u = 2^-11 per weight) and takes the row sum from the same rounded
	// weights, so an output is a weighted mean of V whose weights moved by a
	// factor (1 + e_k), |e_k| <= u. Its error is sum_k w_k e_k (V_k - out),
	// at most u times the mean absolute deviation of V about the output,
	// which is at most half the range of V: u * max |V|. The BF16 tolerance
	// is 5e-3; kF16CopyMax = 8 bounds this term by 2^-8 = 3.9e-3 and leaves
	// the rest for the near-fp32 scores and the fp32 sums. A larger (or
	// non-finite) value is stored as kF16Bad, a NaN pattern that no
	// conversion of a bf16 value produces (its lowest mantissa bit is set,
	// where bf16's 7 mantissa bits fill only fp16's top 7), so the copy
	// itself records which of its elements are unusable, and a buffer
	// holding one runs the exact bf16 path until such rows are overwritten.
	constexpr uint16_t kF16Bad = 0x7e01;
	constexpr float kF16CopyMax = 8.0f;

	__device__ __forceinline__ uint16_t bf16_to_f16_bits(uint32_t b)
	{
		const float f = bf16_bits_to_f32(b);
		if (!(fabsf(f) <= kF16CopyMax)) return kF16Bad;
		return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
	}

	// The change in a buffer's count of kF16Bad elements when `was` is
	// overwritten by `now`.
	__device__ __forceinline__ int bad_delta(uint16_t was, uint16_t now)
	{
		return (now == kF16Bad ? 1 : 0) - (was == kF16Bad ? 1 : 0);
	}

	// Layout of V's fp16 copy: blocked so that the prefill kernels' P.V
	// products read their V^T operand with plain 16-byte LDS reads instead of
	// transposing ones. Rows go in groups of 32 (the buffer is allocated to a
	// whole number of groups); group g holds four blocks of [kv_dim][8]
	// halves. Row p of the group (p = 16 c + s) sits in block 2 c + ((s >> 2)
	// & 1), slot (s & 3) + 4 (s >> 3): block 2 c + h holds rows 16 c + 4 h +
	// j in slots j and rows 16 c + 8 + 4 h + j in slots 4 + j (j < 4), the
	// eight keys whose weights one lane holds for one 16- or 32-key product
	// (the score tiles' key order). So the 16 bytes of column d of a block
	// are one lane's V^T operand, and a 32-row group of one head is four
	// contiguous runs of 16 * head_dim bytes, kv_dim * 16 bytes apart
	// (f16_copy_bytes in kernels.h: the buffer's size).
	__device__ __forceinline__ size_t f16_copy_index(int row, int col, int kv_dim)
	{
		const int p = row & 31;
		const int blk = ((p >> 4) << 1) | ((p >> 2) & 1);
		const int slot = (p & 3) | ((p >> 1) & 4);
		return ((static_cast<size_t>(row >> 5) * 4 + blk) * kv_dim + col) * 8 + slot;
	}

	// Writing the copy for positions pos0 .. pos0 + n_tok - 1 one 16-byte slot
	// set at a time (one thread per block and column: the eight rows' values
	// read coalesced across columns, one 16-byte store) instead of 2 bytes per
	// element, for batches of at least kF16BlockMinTok. Valid when a
	// position's row keeps its place in a 32-row group (rows a multiple of 32,
	// or no wrap) and no row is written twice.
	constexpr int kF16BlockMinTok = 16;
	__host__ __device__ inline bool f16_blocks_ok(int rows, int pos0, int n_tok)
	{
		return n_tok >= kF16BlockMinTok && n_tok <= rows && ((rows & 31) == 0 || pos0 + n_tok <= rows);
	}
	__host__ __device__ inline int f16_block_items(int pos0, int n_tok, int kv_dim)
	{
		return n_tok > 0 ? (((pos0 + n_tok - 1) >> 5) - (pos0 >> 5) + 1) * 4 * kv_dim : 0;
	}
	// Item i of f16_block_items: column i % kv_dim of block (i / kv_dim) % 4 of
	// the 32-position group (pos0 >> 5) + i / (4 kv_dim). src(t, col) gives
	// the BF16 bits of position pos0 + t, which also go to V (row-major, when
	// not null); positions outside the batch keep their slots. Returns the
	// change in the copy's count of kF16Bad elements.
	template <class Src>
	__device__ __forceinline__ int f16_block_item(uint16_t* V16, uint16_t* V, int rows, int kv_dim, int pos0,
	                                              int n_tok, int i, Src src)
	{
		const int d = i % kv_dim, rest = i / kv_dim, blk = rest & 3;
		const int g = (pos0 >> 5) + (rest >> 2);
		const int row0 = (32 * g) % rows; // the group's first row (a multiple of 32)
		const int p0 = 16 * (blk >> 1) + 4 * (blk & 1); // slots 0-3: group rows p0 .. p0 + 3, 4-7: p0 + 8 ..
		const int t0 = 32 * g + p0 - pos0;
		if (t0 + 11 < 0 || t0 >= n_tok || (t0 + 3 < 0 && t0 + 8 >= n_tok)) return 0; // none of the batch
		uint4* dst = reinterpret_cast<uint4*>(V16 + ((static_cast<size_t>(row0 >> 5) * 4 + blk) * kv_dim + d) * 8);
		uint4 w = *dst;
		uint16_t h[8];
		__builtin_memcpy(h, &w, 16);
		int delta = 0;
#pragma unroll
		for (int s = 0; s < 8; ++s)
		{
			const int off = (s & 3) + 8 * (s >> 2), t = t0 + off;
			if (t >= 0 && t < n_tok)
			{
				const uint32_t b = src(t, d);
				if (V) V[static_cast<size_t>(row0 + p0 + off) * kv_dim + d] = static_cast<uint16_t>(b);
				const uint16_t v16 = bf16_to_f16_bits(b);
				delta += bad_delta(h[s], v16);
				h[s] = v16;
			}
		}
		__builtin_memcpy(&w, h, 16);
		*dst = w;
		return delta;
	}

	// Qwen3.5's output gate on one attention output (reference
	// model.cpp:1759-1760, nn_ops.cpp:1731-1742): y * (1 / (1 + e^-g)).
	__device__ __forceinline__ float gated(float y, const float* gate, size_t i)
	{
		return gate ? y * (1.0f / (1.0f + expf(-gate[i]))) : y;
	}

	constexpr float kLog2e = 1.4426950408889634f;
}
