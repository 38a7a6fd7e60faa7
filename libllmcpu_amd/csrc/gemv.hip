// The weight gemvs on either side of nnc's attention (reference
// src/libnnc/nn_ops.h:95-180; model.cpp:1189-1210 picks one by tensor type):
// Y[t][r] = sum_k W[r][k] X[t][k] for up to 16 activation vectors against one
// pass over the weights, W in BF16, in the Q8_0 split layout (int8 q, one
// BF16 scale per 32-column block) or the Q4_S split layout (nibble q, BF16
// scale and bias per block; reference docs/design.md:141-193).
//
// MFMA formulation (v_mfma_f32_16x16x32_bf16): 16 weight rows x 16 tokens per
// product, one 32-column block per k-step. A = the rows' weights of the block
// as bf16, exact for BF16 and for the integer q of Q8_0 (|q| <= 127) and Q4_S
// (0..15). B = X^T split into bf16 hi + lo (x ~= hi + lo to about 16 bits), so
// the product against the exact A is near-fp32 and the accumulation fp32. A
// quantised block's product starts from zero and is scaled into the row's sum
// with the block's scale; Q4_S adds bias * (block sum of x) in a second sum.
//
// Grid: (row groups of kGemvRows = 128, K splits). A work-group of 8
// wavefronts (two work-groups per CU) stages its K range of X^T (hi, lo, and
// for Q4_S the block sums) in LDS once; each wavefront then streams the
// weights of its own 16 rows block by block over the whole range, kAhead<F>
// blocks of loads in flight (BF16: every block of its split, at most 16,
// issued before X^T is staged). With one K split the rows go straight to Y; with
// several, each split writes a partial and a second kernel adds the splits in
// split order, so results are the same run to run.
#include "device_common.h"
#include "kernels.h"

#include <algorithm>

namespace nnchip
{
	namespace
	{
		// Blocks of weights in flight per wavefront of the batch kernel, per
		// layout (a 16-vector Qwen3-4B layer, us, at 8 / 4 / 3 / 2: BF16 91.6 /
		// 87.5 / 87.6 / 89.6, Q8_0 97.6 / 88.9 / 89.5 / 85.7, Q4_S 96.5 / 90.2 /
		// 90.3 / 87.7; 12 was slower still than 8).
		template <int F>
		constexpr int kAhead = F == kGemvBf16 ? 4 : 2;
		// BF16 instead issues every weight load of its K split (at most
		// kGemvBf16Blocks blocks, 16 bytes per lane each) before X^T is staged, and
		// runs its blocks unrolled with no load left to wait for (a 16-vector
		// Qwen3-4B layer 86.9 -> 77.8 us; the quantised layouts, whose loads are
		// 8 and 4 bytes, ran 8 % slower that way: 92.1 and 94.5 us).
		constexpr int kGemvBf16Blocks = 16;
		// 16-byte loads in flight per lane of the one-vector kernel, per layout
		// (a one-vector Qwen3-4B layer, us, at 8 / 6 / 4: BF16 55.7 / 56.1 /
		// 59.2, Q8_0 48.7 / 48.9 / 48.4, Q4_S 51.5 / 50.9 / 48.4; 16 slower).
		template <int F>
		constexpr int kVecAhead = F == kGemvQ4S ? 4 : 8;

		// The matrix holding stacked row `row` and the row's index in it (row
		// uniform over the caller's rows: a row pair or a 16-row tile).
		struct mat_row
		{
			gemv_mat m;
			int r;
		};
		__device__ __forceinline__ mat_row locate(const gemv_params& p, int row)
		{
			const int k = (row >= p.mrow[1]) + (row >= p.mrow[2]);
			const gemv_mat& m = k == 0 ? p.mats[0] : (k == 1 ? p.mats[1] : p.mats[2]);
			return {m, row - (k == 0 ? 0 : (k == 1 ? p.mrow[1] : p.mrow[2]))};
		}

		// MFMA k-slots of a 32-column block: a lane of k-group g holds slots
		// 8 g .. 8 g + 7. For BF16 and Q8_0 slot s is column s. Q4_S packs
		// elements i and i + 16 into byte i, so a lane reading bytes 4 g .. 4 g + 3
		// holds columns 4 g .. 4 g + 3 (low nibbles, slots 8 g .. 8 g + 3) and
		// 16 + 4 g .. 16 + 4 g + 3 (high nibbles, slots 8 g + 4 .. 8 g + 7); X^T is
		// staged in the same slot order.

		// Two fp32 values whose bf16 is exact (integers below 256 in magnitude)
		// -> one packed bf16 pair: the upper halves of their bit patterns.
		__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi)
		{
			return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
		}

		// Eight int8 q (two dwords) -> bf16: u = q + 128 as unsigned bytes,
		// float(u) - 128 = q exactly.
		__device__ __forceinline__ bf16x8 q8_to_bf16x8(uint32_t w0, uint32_t w1)
		{
			u32x4 r;
			const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
			auto byte = [](uint32_t u, int i) { return static_cast<float>((u >> (8 * i)) & 0xffu) - 128.0f; };
			r[0] = pack_hi16(byte(u0, 0), byte(u0, 1));
			r[1] = pack_hi16(byte(u0, 2), byte(u0, 3));
			r[2] = pack_hi16(byte(u1, 0), byte(u1, 1));
			r[3] = pack_hi16(byte(u1, 2), byte(u1, 3));
			return as_bf16x8(r);
		}

		// Four Q4_S bytes -> bf16 slots: low nibbles then high nibbles.
		__device__ __forceinline__ bf16x8 q4_to_bf16x8(uint32_t w)
		{
			u32x4 r;
			const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
			auto byte = [](uint32_t u, int i) { return static_cast<float>((u >> (8 * i)) & 0xffu); };
			r[0] = pack_hi16(byte(lo, 0), byte(lo, 1));
			r[1] = pack_hi16(byte(lo, 2), byte(lo, 3));
			r[2] = pack_hi16(byte(hi, 0), byte(hi, 1));
			r[3] = pack_hi16(byte(hi, 2), byte(hi, 3));
			return as_bf16x8(r);
		}

		template <int F>
		struct a_block
		{
			u32x4 v; // BF16: 8 weights; Q8_0: 8 int8 in v[0..1]; Q4_S: 4 bytes in v[0]
		};

		// Row `row` of W (cols columns), block blk, the lane's k-group grp.
		template <int F>
		__device__ __forceinline__ a_block<F> load_a(const void* W, int cols, int row, int blk, int grp)
		{
			a_block<F> a;
			const size_t base = static_cast<size_t>(row) * cols + 32 * blk;
			if constexpr (F == kGemvBf16)
				a.v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(W) + base + 8 * grp);
			else if constexpr (F == kGemvQ8_0)
			{
				const u32x2 w = *reinterpret_cast<const u32x2*>(static_cast<const int8_t*>(W) + base + 8 * grp);
				a.v = u32x4{w.x, w.y, 0u, 0u};
			}
			else
				a.v = u32x4{*reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(W) + base / 2 + 4 * grp), 0u,
				            0u, 0u};
			return a;
		}

		template <int F>
		__device__ __forceinline__ bf16x8 a_operand(const a_block<F>& a)
		{
			if constexpr (F == kGemvBf16)
				return as_bf16x8(a.v);
			else if constexpr (F == kGemvQ8_0)
				return q8_to_bf16x8(a.v[0], a.v[1]);
			else
				return q4_to_bf16x8(a.v[0]);
		}

		template <int F>
		__global__ __launch_bounds__(4 * kGemvRows) void gemv_kernel(const gemv_params p)
		{
			// Dynamic LDS: X^T hi and lo [block][token][32 slots] (bf16), the 16
			// rows' scales (and biases) [block][16], and the wavefronts' sums.
			extern __shared__ __attribute__((aligned(16))) unsigned char s_raw[];
			const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
			const int col = lane & 15, grp = lane >> 4;
			const int nt = p.n_batch;
			const int split = blockIdx.y;
			const int b0 = split * p.split_blocks;
			const int nblk = min(p.split_blocks, p.cols / 32 - b0); // >= 1
			uint16_t* s_xh = reinterpret_cast<uint16_t*>(s_raw);
			uint16_t* s_xl = s_xh + static_cast<size_t>(p.split_blocks) * nt * 32;
			uint16_t* s_sc = s_xl + static_cast<size_t>(p.split_blocks) * nt * 32;
			uint16_t* s_bi = s_sc + p.split_blocks * kGemvRows;
			float* s_xs = reinterpret_cast<float*>(s_bi + p.split_blocks * kGemvRows); // Q4_S: [block][token] sums of x

			// The work-group's kGemvRows rows; wavefront w takes rows 16 w .. 16 w + 15
			// over every block of the range, kAhead blocks in flight, the first
			// ones while X^T is staged.
			const int row0 = blockIdx.x * kGemvRows + 16 * wave;
			// The tile's matrix (one for all 16 rows) and its rows in it (a tile
			// past the last row has none and only helps stage X^T).
			const int m_rows = max(0, min(16, p.rows - row0)); // (only the last matrix's last tile is short)
			const mat_row mr = locate(p, min(row0, p.rows - 1));
			const int ra = mr.r + min(col, max(m_rows - 1, 0)); // this lane's A row in the matrix (clamped; not stored)
			const int n_mine = m_rows > 0 ? nblk : 0; // blocks of this wavefront
			auto my_block = [&](int i) { return b0 + min(i, max(n_mine - 1, 0)); };
			constexpr int NA = F == kGemvBf16 ? kGemvBf16Blocks : kAhead<F>; // loads in flight
			a_block<F> ab[NA];
#pragma unroll
			for (int j = 0; j < NA; ++j) ab[j] = load_a<F>(mr.m.w, p.cols, ra, min(my_block(j), p.cols / 32 - 1), grp);

			// X^T of the range, four columns per piece (consecutive threads read
			// consecutive 16 bytes of a token's row), loads issued eight at a time.
			const int n_pieces = nblk * nt * 8;
			for (int i0 = 0; i0 < n_pieces; i0 += 4 * kGemvRows * 8)
			{
				float4 xv[8];
#pragma unroll
				for (int u = 0; u < 8; ++u)
				{
					const int i = i0 + threadIdx.x + 4 * kGemvRows * u;
					const int q = i & 7, b = (i >> 3) % nblk, t = (i >> 3) / nblk;
					xv[u] = i < n_pieces ? *reinterpret_cast<const float4*>(p.x + t * p.x_stride + 32 * (b0 + b) + 4 * q)
					                     : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				}
#pragma unroll
				for (int u = 0; u < 8; ++u)
				{
					const int i = i0 + threadIdx.x + 4 * kGemvRows * u;
					if (i >= n_pieces) continue;
					const int q = i & 7, b = (i >> 3) % nblk, t = (i >> 3) / nblk;
					// The piece's first k-slot; its four columns take four consecutive slots.
					const int slot0 = F == kGemvQ4S ? (q < 4 ? 8 * q : 8 * (q - 4) + 4) : 4 * q;
					const uint32_t h0 = cvt_pk_bf16(xv[u].x, xv[u].y), h1 = cvt_pk_bf16(xv[u].z, xv[u].w);
					const uint32_t l0 = cvt_pk_bf16(xv[u].x - bf16_lo(h0), xv[u].y - bf16_hi(h0));
					const uint32_t l1 = cvt_pk_bf16(xv[u].z - bf16_lo(h1), xv[u].w - bf16_hi(h1));
					const size_t at = (static_cast<size_t>(b) * nt + t) * 32 + slot0;
					*reinterpret_cast<u32x2*>(s_xh + at) = u32x2{h0, h1};
					*reinterpret_cast<u32x2*>(s_xl + at) = u32x2{l0, l1};
				}
			}
			const int nb_all = p.cols / 32;
			if constexpr (F == kGemvQ4S)
			{
				// Block sums of x: the caller's, or as the reference evaluates them
				// (reference nn_ops.cpp:1305-1316 under its -ffast-math build:
				// lane j = (x[j] + x[8 + j]) + (x[16 + j] + x[24 + j]), then the
				// lanes pairwise).
				for (int i = threadIdx.x; i < nblk * nt; i += 4 * kGemvRows)
				{
					const int b = i % nblk, t = i / nblk;
					float sum;
					if (p.xsum)
						sum = p.xsum[t * p.xsum_stride + b0 + b];
					else
					{
						const float4* x4 = reinterpret_cast<const float4*>(p.x + t * p.x_stride + 32 * (b0 + b));
						float x[32];
#pragma unroll
						for (int u = 0; u < 8; ++u)
						{
							const float4 v = x4[u];
							x[4 * u] = v.x;
							x[4 * u + 1] = v.y;
							x[4 * u + 2] = v.z;
							x[4 * u + 3] = v.w;
						}
						float l[8];
#pragma unroll
						for (int j = 0; j < 8; ++j) l[j] = (x[j] + x[8 + j]) + (x[16 + j] + x[24 + j]);
						sum = ((l[0] + l[4]) + (l[1] + l[5])) + ((l[2] + l[6]) + (l[3] + l[7]));
					}
					s_xs[b * nt + t] = sum;
				}
			}
			if constexpr (F != kGemvBf16)
			{
				// The work-group's rows' scales (and biases) of the range, [block][row], so
				// a lane reads its four rows with one 8-byte read.
				for (int i = threadIdx.x; i < nblk * kGemvRows; i += 4 * kGemvRows)
				{
					const int r = i / nblk, b = i % nblk;
					const int sr = min(blockIdx.x * kGemvRows + r, p.rows - 1); // stacked row (clamped; not used past the end)
					const mat_row sm = locate(p, sr);
					const size_t src = static_cast<size_t>(sm.r) * nb_all + b0 + b;
					s_sc[b * kGemvRows + r] = sm.m.scales[src];
					if constexpr (F == kGemvQ4S) s_bi[b * kGemvRows + r] = sm.m.biases[src];
				}
			}
			__syncthreads();

			f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f}, acc_b = {0.0f, 0.0f, 0.0f, 0.0f};
			const bf16x8 zero8 = as_bf16x8(u32x4{0u, 0u, 0u, 0u});
			for (int i0 = 0; i0 < n_mine; i0 += NA)
			{
#pragma unroll
				for (int j = 0; j < NA; ++j)
				{
					const int i = i0 + j;
					const int bl = my_block(i) - b0; // block within the range
					const bf16x8 a = a_operand<F>(ab[j]);
					// The next load into this slot, kAhead blocks on (clamped: a
					// load is never under a branch); BF16 has all of its loads out.
					if constexpr (F != kGemvBf16)
						ab[j] = load_a<F>(mr.m.w, p.cols, ra, min(my_block(i + kAhead<F>), nb_all - 1), grp);
					if (i < n_mine) // uniform
					{
						const size_t at = (static_cast<size_t>(bl) * nt + col) * 32 + 8 * grp;
						const bf16x8 xh = col < nt ? *reinterpret_cast<const bf16x8*>(s_xh + at) : zero8;
						const bf16x8 xl = col < nt ? *reinterpret_cast<const bf16x8*>(s_xl + at) : zero8;
						if constexpr (F == kGemvBf16)
						{
							acc = mfma16x16x32(a, xh, acc);
							acc = mfma16x16x32(a, xl, acc);
						}
						else
						{
							f32x4 d = {0.0f, 0.0f, 0.0f, 0.0f};
							d = mfma16x16x32(a, xh, d);
							d = mfma16x16x32(a, xl, d);
							const u32x2 sc = *reinterpret_cast<const u32x2*>(s_sc + bl * kGemvRows + 16 * wave + 4 * grp);
							acc[0] = fmaf(bf16_lo(sc.x), d[0], acc[0]);
							acc[1] = fmaf(bf16_hi(sc.x), d[1], acc[1]);
							acc[2] = fmaf(bf16_lo(sc.y), d[2], acc[2]);
							acc[3] = fmaf(bf16_hi(sc.y), d[3], acc[3]);
							if constexpr (F == kGemvQ4S)
							{
								// The bias term: bias * (block sum of x).
								const u32x2 bi = *reinterpret_cast<const u32x2*>(s_bi + bl * kGemvRows + 16 * wave + 4 * grp);
								const float xs = col < nt ? s_xs[bl * nt + col] : 0.0f;
								acc_b[0] = fmaf(bf16_lo(bi.x), xs, acc_b[0]);
								acc_b[1] = fmaf(bf16_hi(bi.x), xs, acc_b[1]);
								acc_b[2] = fmaf(bf16_lo(bi.y), xs, acc_b[2]);
								acc_b[3] = fmaf(bf16_hi(bi.y), xs, acc_b[3]);
							}
						}
					}
				}
			}

			// Lane (grp, col) holds rows 4 grp + i of token col.
#pragma unroll
			for (int i = 0; i < 4; ++i)
			{
				const int r = 4 * grp + i, t = col;
				const float v = F == kGemvQ4S ? acc[i] + acc_b[i] : acc[i];
				if (r < m_rows && t < nt)
				{
					if (p.n_split == 1)
						mr.m.y[t * mr.m.y_stride + mr.r + r] = v;
					else
						p.part[(static_cast<size_t>(split) * nt + t) * p.rows + row0 + r] = v;
				}
			}
		}

		// One activation vector (the decode gemv) on the VALU: every load is 16
		// contiguous bytes of a weight row (a wavefront reads 1 KB of one row
		// per instruction), x sits in LDS, and each wavefront streams pairs of
		// rows with kVecAhead<F> loads in flight across row boundaries; a row's
		// lane sums meet through DPP and lane swaps.
		template <int F>
		struct vec_shape
		{
			static constexpr int CPL = F == kGemvBf16 ? 8 : (F == kGemvQ8_0 ? 16 : 32); // columns per lane per load
			static constexpr int CW = 64 * CPL; // columns per wavefront load
		};

		template <int F>
		struct vec_item
		{
			u32x4 w; // 16 bytes of the row
			float sc, bi; // the block's scale (Q8_0, Q4_S) and bias (Q4_S)
		};

		// x in LDS for the one-vector kernels. Q4_S (a lane's 32 columns per
		// load, its reads 128 bytes apart in column order: 8-way bank
		// conflicts) keeps it in the order the lanes read it: the four
		// consecutive columns 4 g .. 4 g + 3 of lane l's CPL columns of a
		// CW-column chunk sit at chunk * CW + 256 g + 4 l, so each of a
		// wavefront's 16-byte LDS reads covers 1 KB of consecutive addresses
		// (Qwen3-4B layer, one vector: 58.3 -> 51.6 us), the chunks padded to
		// CW columns and the block sums after them. BF16 and Q8_0 keep column
		// order (the same layout measured no faster for BF16, 6 % slower for
		// Q8_0).
		template <int F>
		constexpr bool kVecLaneOrder = F == kGemvQ4S;

		template <int F>
		__host__ __device__ constexpr int vec_x_floats(int cols)
		{
			return kVecLaneOrder<F> ? (cols + vec_shape<F>::CW - 1) / vec_shape<F>::CW * vec_shape<F>::CW : cols;
		}

		// The lane's dot product of one item (16 bytes of a row at columns
		// c0 ..) with x in LDS.
		template <int F>
		__device__ __forceinline__ float vec_dot(const vec_item<F>& it, int c0, const float* s_x, int cols)
		{
			constexpr int CPL = vec_shape<F>::CPL;
			if (c0 >= cols) return 0.0f;
			const int lane = threadIdx.x & 63;
			// columns c0 + 4 g .. + 3 at xq + GS g
			constexpr int GS = kVecLaneOrder<F> ? 256 : 4;
			const float* xq = kVecLaneOrder<F> ? s_x + (c0 - lane * CPL) + 4 * lane : s_x + c0;
			if constexpr (F == kGemvBf16)
			{
				const float4 x0 = *reinterpret_cast<const float4*>(xq);
				const float4 x1 = *reinterpret_cast<const float4*>(xq + GS);
				float d = 0.0f;
				d = fmaf(bf16_lo(it.w[0]), x0.x, d);
				d = fmaf(bf16_hi(it.w[0]), x0.y, d);
				d = fmaf(bf16_lo(it.w[1]), x0.z, d);
				d = fmaf(bf16_hi(it.w[1]), x0.w, d);
				d = fmaf(bf16_lo(it.w[2]), x1.x, d);
				d = fmaf(bf16_hi(it.w[2]), x1.y, d);
				d = fmaf(bf16_lo(it.w[3]), x1.z, d);
				d = fmaf(bf16_hi(it.w[3]), x1.w, d);
				return d;
			}
			else if constexpr (F == kGemvQ8_0)
			{
				float d = 0.0f;
#pragma unroll
				for (int u = 0; u < 4; ++u)
				{
					const float4 x = *reinterpret_cast<const float4*>(xq + GS * u);
					const uint32_t b = it.w[u] ^ 0x80808080u; // q + 128 per byte
					d = fmaf(static_cast<float>(b & 0xffu) - 128.0f, x.x, d);
					d = fmaf(static_cast<float>((b >> 8) & 0xffu) - 128.0f, x.y, d);
					d = fmaf(static_cast<float>((b >> 16) & 0xffu) - 128.0f, x.z, d);
					d = fmaf(static_cast<float>(b >> 24) - 128.0f, x.w, d);
				}
				return it.sc * d;
			}
			else
			{
				// Byte i of the block: element i (low nibble), i + 16 (high).
				float d = 0.0f;
#pragma unroll
				for (int u = 0; u < 4; ++u)
				{
					const float4 xl = *reinterpret_cast<const float4*>(xq + GS * u); // columns 4 u ..
					const float4 xh = *reinterpret_cast<const float4*>(xq + GS * (4 + u)); // columns 16 + 4 u ..
					const uint32_t b = it.w[u];
					d = fmaf(static_cast<float>(b & 0xfu), xl.x, d);
					d = fmaf(static_cast<float>((b >> 8) & 0xfu), xl.y, d);
					d = fmaf(static_cast<float>((b >> 16) & 0xfu), xl.z, d);
					d = fmaf(static_cast<float>((b >> 24) & 0xfu), xl.w, d);
					d = fmaf(static_cast<float>((b >> 4) & 0xfu), xh.x, d);
					d = fmaf(static_cast<float>((b >> 12) & 0xfu), xh.y, d);
					d = fmaf(static_cast<float>((b >> 20) & 0xfu), xh.z, d);
					d = fmaf(static_cast<float>(b >> 28), xh.w, d);
				}
				return fmaf(it.bi, s_x[vec_x_floats<F>(cols) + c0 / 32], it.sc * d);
			}
		}

		// 16 bytes of row r of matrix m at columns c0 .. (lanes past the row's
		// end re-read its last bytes; their sums are not used), with the
		// block's scale and bias.
		template <int F>
		__device__ __forceinline__ vec_item<F> vec_load(const gemv_mat& m, int r, int c0, int cols)
		{
			constexpr int CPL = vec_shape<F>::CPL;
			const int cc = min(c0, cols - CPL);
			vec_item<F> it;
			const size_t off = static_cast<size_t>(r) * cols + cc;
			if constexpr (F == kGemvBf16)
				it.w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(m.w) + off);
			else if constexpr (F == kGemvQ8_0)
				it.w = *reinterpret_cast<const u32x4*>(static_cast<const int8_t*>(m.w) + off);
			else
				it.w = *reinterpret_cast<const u32x4*>(static_cast<const uint8_t*>(m.w) + off / 2);
			if constexpr (F != kGemvBf16)
			{
				const size_t si = static_cast<size_t>(r) * (cols / 32) + cc / 32;
				it.sc = bf16_bits_to_f32(m.scales[si]);
				if constexpr (F == kGemvQ4S) it.bi = bf16_bits_to_f32(m.biases[si]);
			}
			return it;
		}

		// x into LDS (in the lanes' order for Q4_S, vec_x_floats), and for Q4_S
		// its block sums after it; the caller's barrier follows. Thread t takes elements 4 t .. 4 t + 3
		// of each 1024. Q4_S without the caller's block sums: the eight threads
		// of a block hold its quarters q = t % 8, and three lane exchanges add
		// them in the reference's order (reference nn_ops.cpp:1305-1316 under
		// its -ffast-math build: l_j = (x_j + x_8+j) + (x_16+j + x_24+j), then
		// ((l0 + l4) + (l1 + l5)) + ((l2 + l6) + (l3 + l7))), so x is read once.
		template <int F>
		__device__ __forceinline__ void vec_stage_x(const gemv_params& p, float* s_x)
		{
			constexpr int CW = vec_shape<F>::CW, CPL = vec_shape<F>::CPL;
			const int nb_all = p.cols / 32;
			const int xs = vec_x_floats<F>(p.cols); // the block sums' offset
			const bool own_sums = F == kGemvQ4S && p.xsum == nullptr; // uniform
			for (int i0 = 0; i0 < p.cols; i0 += 1024)
			{
				const int i = i0 + 4 * threadIdx.x;
				const bool ok = i < p.cols; // a block's eight threads agree (cols % 32 == 0)
				const float4 v = ok ? *reinterpret_cast<const float4*>(p.x + i) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				const int rem = i % CW; // lane rem / CPL, group (rem % CPL) / 4 of chunk i / CW
				const int dst = kVecLaneOrder<F> ? (i - rem) + 256 * ((rem % CPL) / 4) + 4 * (rem / CPL) : i;
				if (ok) *reinterpret_cast<float4*>(s_x + dst) = v;
				if (own_sums)
				{
					auto add_from = [](const float4& a, int m) __attribute__((always_inline)) -> float4
					{
						return make_float4(a.x + __shfl_xor(a.x, m), a.y + __shfl_xor(a.y, m), a.z + __shfl_xor(a.z, m),
						                   a.w + __shfl_xor(a.w, m));
					};
					const float4 a = add_from(v, 2); // q = 0: x_j + x_8+j; q = 4: x_16+j + x_24+j (j < 4)
					const float4 l = add_from(a, 4); // q = 0: l_0..3; q = 1: l_4..7
					const float4 u = add_from(l, 1); // q = 0: l_k + l_k+4
					if (ok && (threadIdx.x & 7) == 0) s_x[xs + i / 32] = (u.x + u.y) + (u.z + u.w);
				}
			}
			if (F == kGemvQ4S && !own_sums)
				for (int b = threadIdx.x; b < nb_all; b += 256) s_x[xs + b] = p.xsum[b];
		}

		// The argmax order: (v, r) beats (bv, br) when v is above -inf (NaN never
		// is) and larger, or equal with a smaller row; br = -1 is "none". The
		// smallest row of the largest value wins whatever order rows are met in.
		__device__ __forceinline__ bool argmax_better(float v, int r, float bv, int br)
		{
			return r >= 0 && v > -INFINITY && (br < 0 || v > bv || (v == bv && r < br));
		}

		// ARGMAX (BF16 only): no y; each wavefront keeps its best row and the
		// work-group writes its best (value, row) to p.best[blockIdx.x].
		template <int F, bool ARGMAX = false>
		__global__ __launch_bounds__(256) void gemv_vec_kernel(const gemv_params p)
		{
			static_assert(!ARGMAX || F == kGemvBf16, "argmax of a BF16 gemv only");
			using V = vec_shape<F>;
			constexpr int CPL = V::CPL, CW = V::CW, NA = kVecAhead<F>;
			extern __shared__ __attribute__((aligned(16))) float s_x[]; // x, then (Q4_S) its block sums
			// (wave uniform: every row index below, and the matrix lookup, stays scalar)
			const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

			// Items: for each of this wavefront's row pairs, chunk c of row 0,
			// then of row 1, for every chunk c of CW columns. Two cursors walk
			// them, the loads' (kVecAhead<F> ahead) and the sums': (pair, item within
			// the pair), stepped by one item at a time (no division per item);
			// a pair's matrix is looked up when the load cursor enters it.
			const int nch = (p.cols + CW - 1) / CW;
			const int per_pair = 2 * nch;
			const int gw = blockIdx.x * 4 + wave, n_gw = gridDim.x * 4;
			const int n_pairs = (p.rows + 1) / 2;
			const int my_pairs = gw < n_pairs ? (n_pairs - 1 - gw) / n_gw + 1 : 0;
			const int n_items = my_pairs * per_pair;
			// (A wavefront without rows still takes part in staging x.)
			int l_pi = 0, l_rem = 0; // the next load's pair and item
			gemv_mat l_m = p.mats[0];
			int l_r0 = 0, l_two = 0; // the pair's first row in its matrix; whether it has a second row
			auto enter_pair = [&]() __attribute__((always_inline))
			{
				const int row0 = 2 * (gw + min(l_pi, max(my_pairs - 1, 0)) * n_gw);
				const mat_row mr = locate(p, min(row0, p.rows - 1));
				l_m = mr.m;
				l_r0 = mr.r;
				l_two = row0 + 1 < p.rows;
			};
			enter_pair();
			// The next item's load (past the wavefront's last item: its last item
			// again, so no load is under a branch), then the cursor steps on.
			auto load = [&]() __attribute__((always_inline)) -> vec_item<F>
			{
				const bool past = l_pi >= my_pairs;
				const int rem = past ? per_pair - 1 : l_rem;
				const vec_item<F> it = vec_load<F>(l_m, l_r0 + ((rem & 1) & l_two), (rem >> 1) * CW + lane * CPL, p.cols);
				if (!past && ++l_rem == per_pair)
				{
					l_rem = 0;
					++l_pi;
					if (l_pi < my_pairs) enter_pair();
				}
				return it;
			};
			auto dot = [&](const vec_item<F>& it, int c0) __attribute__((always_inline)) -> float
			{
				return vec_dot<F>(it, c0, s_x, p.cols);
			};

			// The first loads go out before x is staged.
			vec_item<F> ring[NA];
#pragma unroll
			for (int j = 0; j < NA; ++j) ring[j] = load();

			vec_stage_x<F>(p, s_x);
			__syncthreads();

			float acc[2] = {0.0f, 0.0f};
			float best_v = -INFINITY; // ARGMAX: this wavefront's best row so far (lane 0)
			int best_r = -1;
			int u_pi = 0, u_rem = 0; // the next sum's pair and item
			for (int k0 = 0; k0 < n_items; k0 += NA)
			{
#pragma unroll
				for (int j = 0; j < NA; ++j)
				{
					const int k = k0 + j;
					const vec_item<F> it = ring[j];
					ring[j] = load(); // past the end: a repeat, never under a branch
					if (k < n_items) // uniform
					{
						acc[j & 1] += dot(it, (u_rem >> 1) * CW + lane * CPL);
						if (u_rem == per_pair - 1) // the pair's last item: both rows are complete
						{
							const float y0 = wave_sum_dpp(acc[0]), y1 = wave_sum_dpp(acc[1]);
							const int r0 = 2 * (gw + u_pi * n_gw);
							if constexpr (ARGMAX)
							{
								if (r0 == 0 && lane == 0) p.argmax[1] = __builtin_isnan(y0);
								if (argmax_better(y0, r0, best_v, best_r))
								{
									best_v = y0;
									best_r = r0;
								}
								if (r0 + 1 < p.rows && argmax_better(y1, r0 + 1, best_v, best_r))
								{
									best_v = y1;
									best_r = r0 + 1;
								}
							}
							else if (lane == 0)
							{
								const mat_row mr = locate(p, r0); // the pair's matrix (pairs never span two)
								mr.m.y[mr.r] = y0;
								if (r0 + 1 < p.rows) mr.m.y[mr.r + 1] = y1;
							}
							acc[0] = acc[1] = 0.0f;
						}
						if (++u_rem == per_pair)
						{
							u_rem = 0;
							++u_pi;
						}
					}
				}
			}
			if constexpr (ARGMAX)
			{
				// The work-group's best: the four wavefronts' (lane 0's), after x
				// in LDS, then one (value, row) pair per work-group.
				float* s_best = s_x + vec_x_floats<F>(p.cols);
				if (lane == 0)
				{
					s_best[2 * wave] = best_v;
					s_best[2 * wave + 1] = __int_as_float(best_r);
				}
				__syncthreads();
				if (threadIdx.x == 0)
				{
					float bv = -INFINITY;
					int br = -1;
#pragma unroll
					for (int w = 0; w < 4; ++w)
					{
						const float wv = s_best[2 * w];
						const int wr = __float_as_int(s_best[2 * w + 1]);
						if (argmax_better(wv, wr, bv, br))
						{
							bv = wv;
							br = wr;
						}
					}
					p.best[blockIdx.x] = make_float2(bv, __int_as_float(br));
				}
			}
		}

		// The argmax over the work-groups' best pairs: one work-group of 256.
		__global__ __launch_bounds__(256) void gemv_argmax_final_kernel(const gemv_params p, int n_best)
		{
			__shared__ float s_v[256];
			__shared__ int s_r[256];
			float bv = -INFINITY;
			int br = -1;
			for (int i = threadIdx.x; i < n_best; i += 256)
			{
				const float2 b = p.best[i];
				if (argmax_better(b.x, __float_as_int(b.y), bv, br))
				{
					bv = b.x;
					br = __float_as_int(b.y);
				}
			}
			s_v[threadIdx.x] = bv;
			s_r[threadIdx.x] = br;
			__syncthreads();
			for (int h = 128; h > 0; h >>= 1)
			{
				if (static_cast<int>(threadIdx.x) < h && argmax_better(s_v[threadIdx.x + h], s_r[threadIdx.x + h], s_v[threadIdx.x],
				                                     s_r[threadIdx.x]))
				{
					s_v[threadIdx.x] = s_v[threadIdx.x + h];
					s_r[threadIdx.x] = s_r[threadIdx.x + h];
				}
				__syncthreads();
			}
			if (threadIdx.x == 0) p.argmax[0] = s_r[0] >= 0 && !(p.first_sticks && p.argmax[1]) ? s_r[0] : 0;
		}

		// The argmax's first pass over a float vector: each work-group's best
		// (value, row) pair; y[0]'s NaN flag.
		__global__ __launch_bounds__(256) void argmax_part_kernel(const gemv_params p)
		{
			__shared__ float s_v[256];
			__shared__ int s_r[256];
			float bv = -INFINITY;
			int br = -1;
			for (int i = blockIdx.x * 256 + threadIdx.x; i < p.rows; i += gridDim.x * 256)
			{
				const float v = p.mats[0].y[i];
				if (i == 0) p.argmax[1] = __builtin_isnan(v);
				if (argmax_better(v, i, bv, br))
				{
					bv = v;
					br = i;
				}
			}
			s_v[threadIdx.x] = bv;
			s_r[threadIdx.x] = br;
			__syncthreads();
			for (int h = 128; h > 0; h >>= 1)
			{
				if (static_cast<int>(threadIdx.x) < h && argmax_better(s_v[threadIdx.x + h], s_r[threadIdx.x + h], s_v[threadIdx.x],
				                                     s_r[threadIdx.x]))
				{
					s_v[threadIdx.x] = s_v[threadIdx.x + h];
					s_r[threadIdx.x] = s_r[threadIdx.x + h];
				}
				__syncthreads();
			}
			if (threadIdx.x == 0) p.best[blockIdx.x] = make_float2(s_v[0], __int_as_float(s_r[0]));
		}

		// Y[t][r] = the splits' partials summed in split order.
		__global__ void gemv_reduce_kernel(const gemv_params p)
		{
			const size_t n = static_cast<size_t>(p.n_batch) * p.rows;
			for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
			     i += static_cast<size_t>(gridDim.x) * blockDim.x)
			{
				// Eight splits' loads in flight at a time, added in split order.
				float s = 0.0f;
				for (int k0 = 0; k0 < p.n_split; k0 += 8)
				{
					float v[8];
#pragma unroll
					for (int u = 0; u < 8; ++u)
						v[u] = k0 + u < p.n_split ? p.part[static_cast<size_t>(k0 + u) * n + i] : 0.0f;
#pragma unroll
					for (int u = 0; u < 8; ++u)
						if (k0 + u < p.n_split) s = k0 + u == 0 ? v[u] : s + v[u];
				}
				const int t = static_cast<int>(i / p.rows);
				const mat_row mr = locate(p, static_cast<int>(i % p.rows));
				mr.m.y[t * mr.m.y_stride + mr.r] = s;
			}
		}
	}

	void gemv_plan(int rows, int cols, int n_batch, int format, int& n_split, int& split_blocks)
	{
		(void)rows;
		const int nb = cols / 32;
		// As few K splits as the LDS copy of X^T allows (one for a single
		// vector at every nnc shape), the splits equal in size.
		int max_blocks = 1;
		const int cap = format == kGemvBf16 ? kGemvBf16Blocks : nb;
		while (max_blocks < std::min(nb, cap) && gemv_lds_bytes(max_blocks + 1, n_batch) <= gemv_batch_lds(format))
			++max_blocks;
		n_split = (nb + max_blocks - 1) / max_blocks;
		split_blocks = (nb + n_split - 1) / n_split;
	}

	int gemv_vec_groups(int rows)
	{
		const int n_pairs = (rows + 1) / 2;
		return std::max(1, std::min((n_pairs + 3) / 4, 512));
	}

	// LDS of the one-vector kernel: x in the lanes' order (padded to whole
	// chunks), then Q4_S's block sums, or the argmax's eight floats.
	static size_t gemv_vec_lds(int cols, int format)
	{
		const int xf = format == kGemvBf16   ? vec_x_floats<kGemvBf16>(cols)
		               : format == kGemvQ8_0 ? vec_x_floats<kGemvQ8_0>(cols)
		                                     : vec_x_floats<kGemvQ4S>(cols);
		return static_cast<size_t>(xf + std::max(cols / 32, 8)) * 4;
	}

	bool gemv_vec_fits(int cols, int n_batch, int format)
	{
		return n_batch == 1 && gemv_vec_lds(cols, format) <= kGemvLdsBudget;
	}

	bool launch_gemv(const gemv_params& p, hipStream_t stream)
	{
		if (gemv_vec_fits(p.cols, p.n_batch, p.format))
		{
			const size_t lds = gemv_vec_lds(p.cols, p.format);
			const dim3 grid(gemv_vec_groups(p.rows));
			switch (p.format)
			{
			case kGemvBf16: gemv_vec_kernel<kGemvBf16><<<grid, 256, lds, stream>>>(p); return true;
			case kGemvQ8_0: gemv_vec_kernel<kGemvQ8_0><<<grid, 256, lds, stream>>>(p); return true;
			case kGemvQ4S: gemv_vec_kernel<kGemvQ4S><<<grid, 256, lds, stream>>>(p); return true;
			default: return false;
			}
		}
		const dim3 grid((p.rows + kGemvRows - 1) / kGemvRows, p.n_split);
		const size_t lds = gemv_lds_bytes(p.split_blocks, p.n_batch);
		switch (p.format)
		{
		case kGemvBf16: gemv_kernel<kGemvBf16><<<grid, 4 * kGemvRows, lds, stream>>>(p); break;
		case kGemvQ8_0: gemv_kernel<kGemvQ8_0><<<grid, 4 * kGemvRows, lds, stream>>>(p); break;
		case kGemvQ4S: gemv_kernel<kGemvQ4S><<<grid, 4 * kGemvRows, lds, stream>>>(p); break;
		default: return false;
		}
		if (p.n_split > 1)
		{
			const size_t n = static_cast<size_t>(p.n_batch) * p.rows;
			const unsigned g = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 4096));
			gemv_reduce_kernel<<<g, 256, 0, stream>>>(p);
		}
		return true;
	}

	bool launch_gemv_argmax(const gemv_params& p, hipStream_t stream)
	{
		if (p.format != kGemvBf16 || !gemv_vec_fits(p.cols, 1, kGemvBf16)) return false;
		const int groups = gemv_vec_groups(p.rows);
		const size_t lds = gemv_vec_lds(p.cols, kGemvBf16); // x, then the wavefronts' best pairs
		gemv_vec_kernel<kGemvBf16, true><<<groups, 256, lds, stream>>>(p);
		gemv_argmax_final_kernel<<<1, 256, 0, stream>>>(p, groups);
		return true;
	}

	bool launch_argmax(const gemv_params& p, hipStream_t stream)
	{
		const int groups = std::max(1, std::min((p.rows + 1023) / 1024, kArgmaxGroups));
		argmax_part_kernel<<<groups, 256, 0, stream>>>(p);
		gemv_argmax_final_kernel<<<1, 256, 0, stream>>>(p, groups);
		return true;
	}
}
