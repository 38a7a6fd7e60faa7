// Split-K flash-decode for one query token (the n_tok == 1 case of nnc's
// attention core, reference src/libnnc/model.cpp:1731-1749, whose unit of
// work is a (KV head, 256-key block) pair).
//
// Grid: one dimension over (split, head group, token group) (wg_coords). A
// work-group of 4 wavefronts owns a head group (BF16: two KV heads when n_kv
// is even, heads h and h + 2 of a group of four; F32: one) and one
// absolute-aligned range of split_keys keys of the query's span; each head's
// 64-key chunks go to its wavefronts in turn, the next chunk's K and V loads
// in flight while the current one is computed:
//   scores   S^T[key][head] = K . Q^T on MFMA (v_mfma_f32_16x16x32_bf16): the
//            16 keys of a tile are the M rows, loaded straight from HBM in
//            the A-operand layout (16 contiguous bytes per lane; BF16 through
//            range-checked buffer descriptors with the non-temporal hint, a
//            dead chunk's loads aimed past the range so they return zeros
//            without touching memory); the group's query heads are the N
//            columns. Q is split into bf16 hi + lo
//            halves, so the product against the exact bf16 K is near-fp32;
//   softmax  per head (column): the chunk max over keys, exp2 of the
//            log2-scaled scores, a running (m, l) with the usual rescale;
//   P.V      BF16 caches (decode_bf16_kernel): O^T = V^T . P^T on MFMA. The
//            chunk's V rows go to the wavefront's LDS tile and come back
//            transposed (ds_read_b64_tr_b16) as the A operand; P^T, split into
//            bf16 hi + lo, is the B operand straight from the score registers
//            (the key order inside a 32-key step is permuted to match).
//            F32 caches (f32_decode_kernel): on the VALU in fp32, each lane owning
//            consecutive elements of one V row and reading the key's weights
//            for all heads of the group from LDS.
// The four wavefront partials merge in LDS; the work-group's partial
// (o, m, l per head) goes to global scratch, and a second small kernel merges
// the splits of each KV head in split order and writes o / l (0 when l == 0,
// reference nn_ops.cpp:492). The order is fixed, so results are the same run
// to run. A one-token launch over at most kFuseMaxSplits splits merges in
// the split launch instead (fused_merge): the last work-group of each head
// group to finish runs the merge kernel's operations. (An agent-scope
// release in every work-group writes back the XCD's L2: that form measured
// 1.7x slower at 32k keys; the fused merge uses scoped stores and loads
// instead of fences.)
#include "device_common.h"
#include "kernels.h"

#include <type_traits>

namespace nnchip
{
	namespace
	{
		// Shape of the F32 kernel: CH keys per wavefront chunk.
		template <int HD>
		struct f32_shape
		{
			static constexpr int VEC = 4; // elements per 16-byte load
			static constexpr int CH = 4096 / HD; // keys per wave chunk
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

		// KV head hh of head group hg. Pairs take heads two apart, {0, 2},
		// {1, 3}, {4, 6}, ..., when n_kv is a multiple of 4: on this part the
		// 512-byte halves of a 1 KiB span stream at different rates when many
		// work-groups read them (measured at head_dim 128: heads 0, 1, 4, 5
		// of adjacent pairs finished 2.5 us after heads 2, 3, 6, 7 in a 26 us
		// call), and a pair two heads apart reads one of each.
		template <int HPW>
		__device__ __forceinline__ int head_of(int hg, int hh, int n_kv)
		{
			if constexpr (HPW == 2)
				if (n_kv % 4 == 0) return (hg >> 1) * 4 + (hg & 1) + 2 * hh;
			return hg * HPW + hh;
		}

		// Floats per (token, query head) partial, in LDS and in the global
		// scratch: o[head_dim], m (log2 units), l, two unused (16-byte rows).
		template <int HD>
		constexpr int part_pitch() { return HD + 4; }

		// The masked maximum of one chunk's scores for a lane's column (keys
		// cbase + 16 t + 4 (lane / 16) + e in sc[t][e]; each column's keys
		// span the 16-lane rows): keys outside [s0, s1] become -inf. When the
		// chunk lies inside the span of every real column of the wavefront
		// (uniform), the masking changes nothing and is skipped. Columns that
		// are not real (past the batch) hold an empty span; they are masked
		// whenever any masking runs and are never read.
		template <int NT>
		__device__ __forceinline__ float softmax_mask_max(f32x4 (&sc)[NT], int cbase, int s0, int s1, bool real, int ch)
		{
			const int grp = (threadIdx.x & 63) >> 4;
			const bool inside = __builtin_amdgcn_ballot_w64(real && !(cbase >= s0 && cbase + ch - 1 <= s1)) == 0 &&
			                    __builtin_amdgcn_ballot_w64(real) != 0;
			float m = -INFINITY;
			if (inside)
			{
#pragma unroll
				for (int t = 0; t < NT; ++t)
#pragma unroll
					for (int e = 0; e < 4; ++e) m = fmaxf(m, sc[t][e]);
			}
			else
			{
#pragma unroll
				for (int t = 0; t < NT; ++t)
#pragma unroll
					for (int e = 0; e < 4; ++e)
					{
						const int k = cbase + 16 * t + 4 * grp + e;
						const float v = (k >= s0 && k <= s1) ? sc[t][e] : -INFINITY;
						sc[t][e] = v;
						m = fmaxf(m, v);
					}
			}
			m = fmaxf(m, __shfl_xor(m, 16));
			return fmaxf(m, __shfl_xor(m, 32));
		}

		// The running offset of a column's online softmax (log2 units): raised
		// to the chunk's maximum only when that exceeds it by more than
		// kLazyOffset, so most chunks keep it and need no rescale (weights then
		// reach up to 2^kLazyOffset, which the fp32 sums and the bf16 hi + lo
		// split of P carry at full relative precision). Every BF16 decode
		// kernel applies it per column, so a token's bits do not depend on the
		// kernel.
		constexpr float kLazyOffset = 8.0f;
		__device__ __forceinline__ float lazy_offset(float m_run, float m_chunk)
		{
			return m_chunk > m_run + kLazyOffset ? m_chunk : m_run;
		}

		// The P operand of one 32-key half of a chunk (the 8 weights a lane
		// supplies) and its part of the row sum, for O^T += V^T . P^T: P split
		// into bf16 hi + lo against the exact bf16 V (near-fp32), the sum of
		// the fp32 weights, two MFMAs per product. Every BF16 decode kernel
		// goes through these two functions, so a token's bits do not depend on
		// which kernel computes it. (P rounded to fp16 against V's fp16 copy,
		// one MFMA per product, was 0.5 % faster per Qwen3-4B decode call but
		// its error grows with |V|: 2e-2 max-abs where V reaches 400.)
		__device__ __forceinline__ void p_operand(const float (&w)[8], u32x4 (&pb)[2], float& lsum)
		{
#pragma unroll
			for (int e = 0; e < 8; ++e) lsum += w[e];
			bf16x8 hi, lo;
			split_bf16x8(w, hi, lo);
			pb[0] = __builtin_bit_cast(u32x4, hi);
			pb[1] = __builtin_bit_cast(u32x4, lo);
		}

		__device__ __forceinline__ void pv_mfma(f32x4& acc, const u32x4& v, const u32x4 (&pb)[2])
		{
			acc = mfma16x16x32(as_bf16x8(v), as_bf16x8(pb[0]), acc);
			acc = mfma16x16x32(as_bf16x8(v), as_bf16x8(pb[1]), acc);
		}

		// Scores of one 16-key tile against Q split into bf16 hi + lo: the hi
		// products and the lo products each accumulate over d in their own
		// chain, and the two sums are added once. (The one-token kernel puts Q's
		// lo halves in spare MFMA columns and adds the columns instead: the
		// same two chains, the same final addition.)
		template <int KK>
		__device__ __forceinline__ f32x4 scores_hilo(const u32x4 (&k)[KK], const bf16x8 (&qh)[KK], const bf16x8 (&ql)[KK])
		{
			f32x4 sh = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, sl = sh;
#pragma unroll
			for (int kk = 0; kk < KK; ++kk)
			{
				const bf16x8 a = as_bf16x8(k[kk]);
				sh = mfma16x16x32(a, qh[kk], sh);
				sl = mfma16x16x32(a, ql[kk], sl);
			}
			return sh + sl;
		}

		// Device-coherent access to the partials of a fused merge, through a
		// buffer descriptor over the launch's partials. The cache-policy
		// argument 16 sets the sc1 scope bit (device scope): a store with it
		// is written through the XCD's L2 and acknowledged once every XCD can
		// see it, and a load with it bypasses the CU's vector cache and is
		// served from the device-coherent level, never from a stale copy in
		// another XCD's L2.
		constexpr int kAuxDevice = 16;

		__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const decode_params& p, int group_pitch)
		{
			const uint32_t bytes = static_cast<uint32_t>(p.n_tok) * p.n_kv * p.n_split * group_pitch * 4u;
			return __builtin_amdgcn_make_buffer_rsrc(p.part, 0, static_cast<int>(bytes), 0x00020000);
		}

		__device__ __forceinline__ void store_device(__amdgpu_buffer_rsrc_t r, uint32_t off, float4 v)
		{
			__builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kAuxDevice);
		}

		__device__ __forceinline__ void store_device(__amdgpu_buffer_rsrc_t r, uint32_t off, float2 v)
		{
			__builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, off, 0, kAuxDevice);
		}

		__device__ __forceinline__ f32x4 load_device4(__amdgpu_buffer_rsrc_t r, uint32_t off)
		{
			return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxDevice));
		}

		__device__ __forceinline__ float2 load_device2(__amdgpu_buffer_rsrc_t r, uint32_t off)
		{
			return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kAuxDevice));
		}

		// The fused merge of head group hg's splits (one-token launches,
		// fused_merge_on). Each thread has stored its share of the
		// work-group's partial with device-scope stores; it waits until they
		// are acknowledged (s_waitcnt vmcnt(0): on gfx9 stores count there),
		// so after the barrier the whole partial is visible on every XCD.
		// One thread then counts the work-group in with a device-scope atomic
		// add; the work-group that brings the count to n_split is the last of
		// its group, every other partial is then visible, and it resets the
		// count to zero for the next launch and merges. Each thread of the
		// last work-group takes float4 columns of the group's (KV head, query
		// head) outputs, loads the column of every split at once and
		// repeats merge_splits' operations:
		// per part (splits with (absolute split number) % PARTS == part) the
		// largest m, then the ascending-split sums against it, then the parts
		// in order against the largest of all. A token therefore gets the
		// same bits from either merge.
		template <int HD, int G, int W, int HPW>
		__device__ __forceinline__ void fused_merge(const decode_params& p, __amdgpu_buffer_rsrc_t rs, int tok, int hg)
		{
			__shared__ int s_last;
			asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
			__syncthreads();
			if (threadIdx.x == 0)
			{
				unsigned* c = p.counts + hg;
				const unsigned prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
				const bool last = prev == static_cast<unsigned>(p.n_split - 1);
				if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
				s_last = last ? 1 : 0;
			}
			__syncthreads();
			if (!s_last) return;

			// F register slots: the splits, and at least one per part (a
			// part's result is kept in the slot of its first split; a part
			// past the last split has none and keeps m = -inf, o = l = 0).
			constexpr int PL = part_pitch<HD>(), Q4 = HD / 4, PARTS = 1024 / HD;
			constexpr int F = PARTS > kFuseMaxSplits ? PARTS : kFuseMaxSplits;
			const int ns = p.n_split, a0 = p.split_base / p.split_keys;
			const uint32_t sstride = G * PL * 4u;
			for (int idx = threadIdx.x; idx < HPW * G * Q4; idx += 64 * W)
			{
				const int hh = idx / (G * Q4), h = (idx / Q4) % G, d4 = idx % Q4;
				const int kvh = head_of<HPW>(hg, hh, p.n_kv);
				const uint32_t base = ((static_cast<uint32_t>(tok) * p.n_kv + kvh) * ns * G + h) * PL * 4u;
				f32x4 o[F];
				float2 ml[F];
#pragma unroll
				for (int u = 0; u < F; ++u)
				{
					if (u < ns)
					{
						const uint32_t sp = base + static_cast<uint32_t>(u) * sstride;
						o[u] = load_device4(rs, sp + 16u * d4);
						ml[u] = load_device2(rs, sp + 4u * HD);
					}
				}
				// Split u belongs to class u % PARTS, and class k to part
				// (a0 + k) % PARTS: the classes are the parts, with each
				// class's splits at fixed register indices. Per class: its
				// largest m, then its ascending-split sums against it, kept in
				// slot k (its first split, already consumed).
#pragma unroll
				for (int k = 0; k < PARTS; ++k)
				{
					float mk = -INFINITY;
#pragma unroll
					for (int u = k; u < F; u += PARTS)
						if (u < ns) mk = fmaxf(mk, ml[u].x);
					const float m_use = mk == -INFINITY ? 0.0f : mk;
					f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
					float L = 0.0f;
#pragma unroll
					for (int u = k; u < F; u += PARTS)
					{
						if (u < ns)
						{
							const float f = fast_exp2(ml[u].x - m_use);
							acc.x = fmaf(o[u].x, f, acc.x);
							acc.y = fmaf(o[u].y, f, acc.y);
							acc.z = fmaf(o[u].z, f, acc.z);
							acc.w = fmaf(o[u].w, f, acc.w);
							L = fmaf(ml[u].y, f, L);
						}
					}
					o[k] = acc;
					ml[k] = make_float2(mk, L);
				}
				float M = -INFINITY;
#pragma unroll
				for (int k = 0; k < PARTS; ++k) M = fmaxf(M, ml[k].x);
				const float M_use = M == -INFINITY ? 0.0f : M;
				// Then the parts in order 0, 1, ...: part j is class
				// (j + c) % PARTS, so the classes go c, c + 1, ..., then 0 ..
				// c - 1 (c is uniform).
				const int c = (PARTS - a0 % PARTS) % PARTS;
				float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				float lt = 0.0f;
				auto add_part = [&](int k) __attribute__((always_inline))
				{
					const float f = fast_exp2(ml[k].x - M_use);
					r.x = fmaf(o[k].x, f, r.x);
					r.y = fmaf(o[k].y, f, r.y);
					r.z = fmaf(o[k].z, f, r.z);
					r.w = fmaf(o[k].w, f, r.w);
					lt = fmaf(ml[k].y, f, lt);
				};
#pragma unroll
				for (int k = 0; k < PARTS; ++k)
					if (k >= c) add_part(k);
#pragma unroll
				for (int k = 0; k < PARTS; ++k)
					if (k < c) add_part(k);
				const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
				const size_t oi = (static_cast<size_t>(tok) * p.n_head + kvh * G + h) * HD + 4 * d4;
				float4 out;
				out.x = gated(r.x * inv, p.gate, oi);
				out.y = gated(r.y * inv, p.gate, oi + 1);
				out.z = gated(r.z * inv, p.gate, oi + 2);
				out.w = gated(r.w * inv, p.gate, oi + 3);
				*reinterpret_cast<float4*>(p.out + oi) = out;
			}
		}

		// The work-group's result from its wavefronts' partials in s_wpart
		// (o[head_dim], m, l per column, per wavefront). The work-group holds
		// the HPW KV heads of head group hg (head_of); wavefront w works for
		// head w % HPW of the group as its lane w / HPW, and a head's lanes
		// merge in lane order. Column c is query head c % G of token
		// tok0 + c / G; the first n_cols columns are filled. With several
		// splits the result is the split's partial; with one it is
		// o * (1 / l), the expression the split merge ends with, so a token
		// gets the same bits either way. Each thread takes four consecutive
		// elements of one column. (Wavefront w's partial of column c starts at
		// s_wpart + w * wstride + c * part_pitch<HD>().)
		template <int HD, int G, int W, int HPW, bool FUSE = true>
		__device__ __forceinline__ void write_wg_result(const decode_params& p, const float* s_wpart, int wstride,
		                                                int tok0, int n_cols, int split, int hg)
		{
			constexpr int PL = part_pitch<HD>(), LPH = W / HPW, kThreads = 64 * W, Q4 = HD / 4;
			const bool single = p.n_split == 1, fused = FUSE && fused_merge_on(p);
			const __amdgpu_buffer_rsrc_t rs = part_rsrc(p, G * PL);
			for (int idx = threadIdx.x; idx < HPW * n_cols * Q4; idx += kThreads)
			{
				const int hh = idx / (n_cols * Q4), c = (idx / Q4) % n_cols, d = 4 * (idx % Q4);
				const int tok = tok0 + c / G, h = c % G, kvh = head_of<HPW>(hg, hh, p.n_kv);
				float mw[LPH], f[LPH];
				float m = -INFINITY;
#pragma unroll
				for (int l = 0; l < LPH; ++l)
				{
					mw[l] = s_wpart[(l * HPW + hh) * wstride + c * PL + HD];
					m = fmaxf(m, mw[l]);
				}
				const float m_use = m == -INFINITY ? 0.0f : m;
#pragma unroll
				for (int l = 0; l < LPH; ++l) f[l] = fast_exp2(mw[l] - m_use);
				float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				float l_sum = 0.0f;
#pragma unroll
				for (int l = 0; l < LPH; ++l)
				{
					const float* wp = s_wpart + (l * HPW + hh) * wstride + c * PL;
					const float4 v = *reinterpret_cast<const float4*>(wp + d);
					r.x = fmaf(v.x, f[l], r.x);
					r.y = fmaf(v.y, f[l], r.y);
					r.z = fmaf(v.z, f[l], r.z);
					r.w = fmaf(v.w, f[l], r.w);
					l_sum = fmaf(wp[HD + 1], f[l], l_sum);
				}
				if (fused)
				{
					const uint32_t off =
						(((static_cast<uint32_t>(tok) * p.n_kv + kvh) * p.n_split + split) * G * PL + h * PL) * 4u;
					store_device(rs, off + 4u * d, r);
					if (d == 0) store_device(rs, off + 4u * HD, make_float2(m, l_sum));
				}
				else if (!single)
				{
					float* gpart = p.part + ((static_cast<size_t>(tok) * p.n_kv + kvh) * p.n_split + split) * G * PL + h * PL;
					*reinterpret_cast<float4*>(gpart + d) = r;
					if (d == 0) *reinterpret_cast<float2*>(gpart + HD) = make_float2(m, l_sum);
				}
				else
				{
					const float inv = l_sum > 0.0f ? 1.0f / l_sum : 0.0f;
					const size_t oi = (static_cast<size_t>(tok) * p.n_head + kvh * G + h) * HD + d;
					float4 o;
					o.x = gated(r.x * inv, p.gate, oi);
					o.y = gated(r.y * inv, p.gate, oi + 1);
					o.z = gated(r.z * inv, p.gate, oi + 2);
					o.w = gated(r.w * inv, p.gate, oi + 3);
					*reinterpret_cast<float4*>(p.out + oi) = o;
				}
			}
			if (fused) fused_merge<HD, G, W, HPW>(p, rs, tok0, hg);
		}

		// A merge work-group takes 1 / SLICES of one (token, query head)'s
		// HD / 4 float4 columns of o: COLS columns times PARTS parts of the
		// splits, 256 / SLICES threads.
		template <int HD, int SLICES>
		struct merge_lds
		{
			static constexpr int PARTS = 1024 / HD, COLS = HD / 4 / SLICES, THREADS = COLS * PARTS;
			float4 o[PARTS][COLS];
			float ls[PARTS], ms[PARTS];
		};

		// Merges the n_split partials of one (token, query head) and writes
		// o * (1 / l) (0 when l == 0, reference nn_ops.cpp:492), columns
		// COLS * slice .. + COLS - 1 of it. Lane t owns float4 column
		// COLS * slice + t % COLS of o for the splits of part t / COLS, whose
		// o, m and l it loads together (B splits per batch: 16, or 32 when a
		// part has more than 16), so the common case is one round trip to
		// memory and one barrier. Every element goes through the same
		// operations whatever SLICES and B are.
		// (For one token, four one-wavefront work-groups per head spread the
		// reads over more CUs than one 256-thread work-group: 0.5 us less per
		// call at 64 splits; for 16 tokens they are 2.9 us slower.) A split belongs to part (its absolute number,
		// split_base / split_keys + s) % PARTS; a part sums its splits in
		// ascending order against its own largest m, then the parts are summed
		// in order, each scaled by 2^(its m - the largest). A split outside
		// the token's span holds m = -inf, l = 0, o = 0 and adds exact zeros,
		// and the parts are fixed by the absolute split grid, so a token's
		// result depends only on its own splits, whatever else the launch
		// covered.
		template <int HD, int G, int SLICES, int B>
		__device__ __forceinline__ void merge_splits(const decode_params& p, int tok, int qh, int slice,
		                                             merge_lds<HD, SLICES>& sh)
		{
			using S = merge_lds<HD, SLICES>;
			constexpr int PL = part_pitch<HD>(), COLS = S::COLS, PARTS = S::PARTS;
			const int kvh = qh / G, h = qh % G;
			const int ns = p.n_split;
			const int c = threadIdx.x % COLS, part = threadIdx.x / COLS, d4 = COLS * slice + c;
			const size_t sstride = static_cast<size_t>(G) * PL;
			const float* hp = p.part + ((static_cast<size_t>(tok) * p.n_kv + kvh) * ns * G + h) * PL;
			// This part's splits: s_first, s_first + PARTS, ... below ns.
			const int a0 = p.split_base / p.split_keys;
			const int s_first = ((part - a0 % PARTS) + PARTS) % PARTS;
			const int n_mine = s_first < ns ? (ns - 1 - s_first) / PARTS + 1 : 0;

			// A batch of B of them (indices clamped to a valid split; the ones
			// past the part's last are not used).
			float4 o[B];
			float2 ml[B];
			auto load_batch = [&](int b0) __attribute__((always_inline))
			{
#pragma unroll
				for (int u = 0; u < B; ++u)
				{
					const float* sp = hp + min(s_first + PARTS * (b0 + u), ns - 1) * sstride;
					o[u] = *reinterpret_cast<const float4*>(sp + 4 * d4);
					ml[u] = *reinterpret_cast<const float2*>(sp + HD);
				}
			};
			// The part's largest m: the first batch's, then the further
			// splits' in batches of B independent loads (one round trip each).
			load_batch(0);
			float mp = -INFINITY;
#pragma unroll
			for (int u = 0; u < B; ++u)
				if (u < n_mine) mp = fmaxf(mp, ml[u].x);
			for (int b0 = B; b0 < n_mine; b0 += B)
			{
				float mb[B];
#pragma unroll
				for (int u = 0; u < B; ++u) mb[u] = hp[min(s_first + PARTS * (b0 + u), ns - 1) * sstride + HD];
#pragma unroll
				for (int u = 0; u < B; ++u)
					if (b0 + u < n_mine) mp = fmaxf(mp, mb[u]);
			}
			const float m_use = mp == -INFINITY ? 0.0f : mp;
			float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
			float L = 0.0f;
			for (int b0 = 0; b0 < n_mine; b0 += B)
			{
				if (b0 > 0) load_batch(b0);
#pragma unroll
				for (int u = 0; u < B; ++u)
				{
					if (b0 + u < n_mine)
					{
						const float f = fast_exp2(ml[u].x - m_use);
						acc.x = fmaf(o[u].x, f, acc.x);
						acc.y = fmaf(o[u].y, f, acc.y);
						acc.z = fmaf(o[u].z, f, acc.z);
						acc.w = fmaf(o[u].w, f, acc.w);
						L = fmaf(ml[u].y, f, L);
					}
				}
			}
			sh.o[part][c] = acc;
			if (c == 0)
			{
				sh.ls[part] = L;
				sh.ms[part] = mp;
			}
			__syncthreads();
			if (part == 0)
			{
				float M = sh.ms[0];
#pragma unroll
				for (int j = 1; j < PARTS; ++j) M = fmaxf(M, sh.ms[j]);
				const float M_use = M == -INFINITY ? 0.0f : M;
				float4 r = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
				float lt = 0.0f;
#pragma unroll
				for (int j = 0; j < PARTS; ++j)
				{
					const float f = fast_exp2(sh.ms[j] - M_use);
					const float4 v = sh.o[j][c];
					r.x = fmaf(v.x, f, r.x);
					r.y = fmaf(v.y, f, r.y);
					r.z = fmaf(v.z, f, r.z);
					r.w = fmaf(v.w, f, r.w);
					lt = fmaf(sh.ls[j], f, lt);
				}
				const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
				const size_t oi = (static_cast<size_t>(tok) * p.n_head + qh) * HD + 4 * d4;
				float4 out;
				out.x = gated(r.x * inv, p.gate, oi);
				out.y = gated(r.y * inv, p.gate, oi + 1);
				out.z = gated(r.z * inv, p.gate, oi + 2);
				out.w = gated(r.w * inv, p.gate, oi + 3);
				*reinterpret_cast<float4*>(p.out + oi) = out;
			}
		}

		// The split merge, launched after the split kernel: SLICES work-groups
		// per (query head, token). (A merge inside the split launch, by extra
		// work-groups that wait on per-head counts and read the partials with
		// device-coherent loads, measured slower: 35 vs 32 us per call at 32k
		// keys, the coherent loads and the polling being slower than the
		// launch boundary.)
		template <int HD, int G, int SLICES, int B>
		__global__ __launch_bounds__(256 / SLICES) void decode_merge_kernel(const decode_params p)
		{
			__shared__ merge_lds<HD, SLICES> sh;
			merge_splits<HD, G, SLICES, B>(p, blockIdx.y, blockIdx.x / SLICES, blockIdx.x % SLICES, sh);
		}

		// The merge over (n_kv * G * SLICES, n_tok) work-groups, 32 splits per
		// batch when a part has more than 16 (one round trip fewer per 32).
		template <int HD, int G, int SLICES>
		void launch_merge(const decode_params& p, int n_tok, hipStream_t stream)
		{
			constexpr int PARTS = 1024 / HD;
			const dim3 grid(p.n_kv * G * SLICES, n_tok);
			if (p.n_split > 16 * PARTS)
				decode_merge_kernel<HD, G, SLICES, 32><<<grid, merge_lds<HD, SLICES>::THREADS, 0, stream>>>(p);
			else
				decode_merge_kernel<HD, G, SLICES, 16><<<grid, merge_lds<HD, SLICES>::THREADS, 0, stream>>>(p);
		}

		// F32 K/V: scores on MFMA with both operands split into bf16 hi + lo
		// (near-fp32), P.V on the VALU in fp32.
		template <int HD, int G>
		__global__ __launch_bounds__(256) void f32_decode_kernel(const decode_params p)
		{
			constexpr int W = 4, kWaves = W;
			using S = f32_shape<HD>;
			constexpr int CH = S::CH, NT = S::NT, KK = S::KK, VEC = S::VEC, LPK = S::LPK, KPL = S::KPL, NV = S::NV;
			constexpr int PW = part_pitch<HD>();

			__shared__ float s_p[kWaves][CH][16]; // weights: [wave][key][head]
			__shared__ float s_alpha[kWaves][16];
			__shared__ __attribute__((aligned(16))) float s_wpart[kWaves][G][PW];

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: keeps chunk control flow scalar
			const int col = lane & 15; // head within the group (MFMA N column)
			const int grp = lane >> 4; // lane group (MFMA K slice / D row quad)
			const int kvh = blockIdx.y;
			const int split = blockIdx.x;
			const int tok = blockIdx.z;

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

			u32x4 kreg[NT][KK][2];
			u32x4 vreg[NV];
			auto chunk_bounds = [&](int c, int& cbase, int& clo, int& chi, int& rb) __attribute__((always_inline))
			{
				cbase = sbase + c * CH;
				clo = max(s0, cbase);
				chi = min(s1, cbase + CH - 1);
				rb = clo < p.rows ? clo : clo % p.rows; // (no division unless the buffer is a ring that wrapped)
			};
			auto load_k = [&](int cbase, int clo, int chi, int rb) __attribute__((always_inline))
			{
#pragma unroll
				for (int t = 0; t < NT; ++t)
				{
					const int k = min(max(cbase + 16 * t + col, clo), chi);
					const size_t row = static_cast<size_t>(ring_row(k, clo, rb, p.rows));
					const float* kp = static_cast<const float*>(p.K) + row * p.kv_dim + head_off + 8 * grp;
#pragma unroll
					for (int kk = 0; kk < KK; ++kk)
					{
						kreg[t][kk][0] = load_stream(kp + 32 * kk);
						kreg[t][kk][1] = load_stream(kp + 32 * kk + 4);
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
					vreg[j] = load_stream(static_cast<const float*>(p.V) + row * p.kv_dim + head_off + VEC * (lane % LPK));
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
						float x[8];
#pragma unroll
						for (int j = 0; j < 4; ++j)
						{
							x[j] = __uint_as_float(kreg[t][kk][0][j]);
							x[4 + j] = __uint_as_float(kreg[t][kk][1][j]);
						}
						bf16x8 khi, klo;
						split_bf16x8(x, khi, klo);
						acc[t] = mfma16x16x32(khi, qhi[kk], acc[t]);
						acc[t] = mfma16x16x32(khi, qlo[kk], acc[t]);
						acc[t] = mfma16x16x32(klo, qhi[kk], acc[t]);
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
#pragma unroll
					for (int u = 0; u < VEC; ++u) v[u] = __uint_as_float(vreg[j][u]);
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

			write_wg_result<HD, G, W, 1>(p, &s_wpart[0][0][0], G * PW, tok, G, split, kvh);
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

		// K/V rows are read through buffer descriptors over the whole layer
		// buffer (the host keeps a BF16 buffer under 2 GiB) with the
		// non-temporal hint. A load past the wavefront's last chunk gets an
		// offset past every buffer: the range check returns zeros without a
		// memory access, so loads need no branch around them.
		constexpr int kBufferFlags = 0x00020000; // descriptor word 3: raw 32-bit data
		constexpr int kAuxStream = 2; // cache policy bits: nt
		constexpr uint32_t kDeadOffset = 0x80000000u;

		__device__ __forceinline__ __amdgpu_buffer_rsrc_t layer_rsrc(const void* base, uint32_t bytes)
		{
			return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufferFlags);
		}

		__device__ __forceinline__ u32x4 load_rows(__amdgpu_buffer_rsrc_t r, uint32_t off)
		{
			return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kAuxStream);
		}

		// One chunk's K rows (the MFMA A operand) and V rows (as loaded, for
		// the wavefront's LDS tile).
		template <int NT, int KK, int NV>
		struct chunk_regs
		{
			u32x4 k[NT][KK];
			u32x4 v[NV];
		};

		// The work-group's (head group, split, token group) from its linear
		// index among nx splits, ny head groups and nz token groups. One
		// token: the head groups of a
		// split are adjacent in dispatch order (linear index = head group
		// fastest), so each split's rows are read as whole runs of
		// HPW * head_dim elements by neighbouring work-groups. Several token
		// groups: those of one (split, head group) go to one XCD in
		// consecutive slots (work-groups are dealt to the XCDs round-robin by
		// linear index), so they stream the same K/V rows through one L2.
		__device__ __forceinline__ void wg_coords(int lin, int nx, int ny, int nz, int& hg, int& split, int& zg)
		{
			const int nxy = nx * ny;
			if (nz > 1 && nxy % 8 == 0)
			{
				const int xcd = lin % 8, slot = lin / 8;
				zg = slot % nz;
				const int pair = 8 * (slot / nz) + xcd;
				hg = pair % ny;
				split = pair / ny;
			}
			else
			{
				zg = lin / nxy;
				hg = (lin % nxy) % ny;
				split = (lin % nxy) / ny;
			}
		}

		// BF16 K/V: both products on MFMA.
		//   S^T = K . Q^T     on MFMA, Q split into bf16 hi + lo.
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
		// Loads run DEPTH chunks ahead in DEPTH register sets: a chunk's K
		// registers are reissued (for the chunk DEPTH ahead) as soon as its
		// scores are done, its V registers as soon as they are in LDS.
		template <int HD, int G, int W, int CHK, int T, int HPW>
		__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(1, 1))) void decode_bf16_kernel(
			const decode_params p)
		{
			using S = bf16_shape<HD, CHK>;
			constexpr int CH = S::CH, NT = S::NT, NC = S::NC, KK = S::KK, DB = S::DB, LPK = S::LPK, KPL = S::KPL,
			              NV = S::NV, VPITCH = S::VPITCH;
			constexpr int PW = part_pitch<HD>(), LPH = W / HPW;
			static_assert(T >= 1 && T * G <= 16, "tokens per work-group");
			static_assert(HPW >= 1 && W % HPW == 0, "heads per work-group");
			constexpr int DEPTH = 1; // chunks of K and V in flight per wavefront (register sets; 2 measured slower)

			__shared__ __attribute__((aligned(16))) uint16_t s_v[W][CH * VPITCH];
			__shared__ __attribute__((aligned(16))) float s_wpart[W][T * G][PW];

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: keeps chunk control flow scalar
			const int col = lane & 15;
			const int grp = lane >> 4;
			const int hh = wave % HPW, hlane = wave / HPW; // this wavefront's head in the work-group, its lane
			const int n_hg = p.n_kv / HPW, n_zg = (p.n_tok + T - 1) / T;
			int hg, split, zg;
			if constexpr (T == 1)
			{
				// One token: a (head group, split) grid, head groups fastest in
				// dispatch order as wg_coords deals them, without its divisions.
				hg = blockIdx.x;
				split = blockIdx.y;
				zg = 0;
				(void)n_zg;
			}
			else
				wg_coords(blockIdx.x, p.n_split, n_hg, n_zg, hg, split, zg);
			const int kvh = head_of<HPW>(hg, hh, p.n_kv);
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
			const bool col_real = tt < n_tt;
			const int col_s0 = col_real ? max(first, sbase) : 1;
			const int col_s1 = col_real ? min(last, send) : 0;
			int f0, l0, fL, lL;
			attn_span(p.causal, p.window, p.pos0 + tok0, p.n_seq, f0, l0);
			attn_span(p.causal, p.window, p.pos0 + tok0 + n_tt - 1, p.n_seq, fL, lL);
			const int s0 = max(f0, sbase);
			const int s1 = min(lL, send);
			const uint32_t row_bytes = static_cast<uint32_t>(p.kv_dim) * 2;
			const __amdgpu_buffer_rsrc_t rk = layer_rsrc(p.K, static_cast<uint32_t>(p.rows) * row_bytes);
			const __amdgpu_buffer_rsrc_t rv = layer_rsrc(p.V, static_cast<uint32_t>(p.rows) * row_bytes);
			const uint32_t k_col = static_cast<uint32_t>(kvh) * HD * 2 + 16 * grp; // + 64 kk
			const uint32_t v_col = static_cast<uint32_t>(kvh) * HD * 2 + 16 * (lane % LPK);
			uint16_t* vt = s_v[wave];

			// The head's chunks of the split go to its lanes in turn.
			const int c_first = s0 <= s1 ? (s0 - sbase) / CH : 0;
			const int c_last = s0 <= s1 ? (s1 - sbase) / CH : -1;
			const int c_wave = c_first + ((hlane - c_first % LPH) + LPH) % LPH;
			const int n_wchunks = c_wave <= c_last ? (c_last - c_wave) / LPH + 1 : 0; // uniform

			auto chunk_bounds = [&](int c, int& cbase, int& clo, int& chi, int& rb) __attribute__((always_inline))
			{
				cbase = sbase + c * CH;
				clo = max(s0, cbase);
				chi = min(s1, cbase + CH - 1);
				rb = clo < p.rows ? clo : clo % p.rows; // (no division unless the buffer is a ring that wrapped)
			};
			using regs = chunk_regs<NT, KK, NV>;
			// The i-th chunk of the wavefront (dead past its last one).
			auto load_k = [&](regs& X, int i) __attribute__((always_inline))
			{
				const bool live = i < n_wchunks;
				int cbase, clo, chi, rb;
				chunk_bounds(c_wave + i * LPH, cbase, clo, chi, rb);
#pragma unroll
				for (int t = 0; t < NT; ++t)
				{
					const int k = min(max(cbase + 16 * t + col, clo), chi);
					const uint32_t off = live ? static_cast<uint32_t>(ring_row(k, clo, rb, p.rows)) * row_bytes + k_col
					                          : kDeadOffset;
#pragma unroll
					for (int kk = 0; kk < KK; ++kk) X.k[t][kk] = load_rows(rk, off + 64 * kk);
				}
			};
			// Load j: key j * KPL + lane / LPK, elements 8 * (lane % LPK) .. + 8.
			auto load_v = [&](regs& X, int i) __attribute__((always_inline))
			{
				const bool live = i < n_wchunks;
				int cbase, clo, chi, rb;
				chunk_bounds(c_wave + i * LPH, cbase, clo, chi, rb);
#pragma unroll
				for (int j = 0; j < NV; ++j)
				{
					const int k = min(max(cbase + j * KPL + lane / LPK, clo), chi);
					X.v[j] = load_rows(rv, live ? static_cast<uint32_t>(ring_row(k, clo, rb, p.rows)) * row_bytes + v_col
					                            : kDeadOffset);
				}
			};

			// Q first (its loads return before the K/V rows issued after them),
			// then the first two chunks of K and V, then Q^T as the B operand,
			// scaled into log2 units and split into bf16 hi + lo. One token
			// (PACK): column c < G holds head c's hi half and column G + c its lo
			// half, so a score takes one MFMA per 32 elements of d (the columns
			// are added after); columns from 2G on are zero.
			constexpr bool PACK = T == 1;
			static_assert(!PACK || 2 * G <= 16, "packed columns");
			const bool q_ok = PACK ? col < 2 * G : tt < n_tt;
			const float* qp =
				p.q + (static_cast<size_t>(tok0 + (PACK || !q_ok ? 0 : tt)) * p.n_head + kvh * G + col % G) * HD + 8 * grp;
			float4 qa[KK], qb[KK];
#pragma unroll
			for (int kk = 0; kk < KK; ++kk)
			{
				qa[kk] = *reinterpret_cast<const float4*>(qp + 32 * kk);
				qb[kk] = *reinterpret_cast<const float4*>(qp + 32 * kk + 4);
			}
			regs X0, X1;
			load_k(X0, 0);
			load_v(X0, 0);
			if constexpr (DEPTH == 2)
			{
				load_k(X1, 1);
				load_v(X1, 1);
			}
			bf16x8 qhi[KK], qlo[KK];
#pragma unroll
			for (int kk = 0; kk < KK; ++kk)
			{
				const float sq = p.qscale;
				float x[8] = {qa[kk].x * sq, qa[kk].y * sq, qa[kk].z * sq, qa[kk].w * sq,
				              qb[kk].x * sq, qb[kk].y * sq, qb[kk].z * sq, qb[kk].w * sq};
#pragma unroll
				for (int j = 0; j < 8; ++j) x[j] = q_ok ? x[j] : 0.0f;
				split_bf16x8(x, qhi[kk], qlo[kk]);
				if constexpr (PACK)
					if (col >= G) qhi[kk] = qlo[kk]; // this lane's B operand is qhi
			}

			float m_run = -INFINITY, l_run = 0.0f;
			f32x4 acc_o[DB];
#pragma unroll
			for (int db = 0; db < DB; ++db) acc_o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

			// The wavefront's i-th chunk from X; X is then reloaded with chunk i + DEPTH.
			auto chunk = [&](regs& X, int i) __attribute__((always_inline))
			{
				int cbase, clo, chi, rb;
				chunk_bounds(c_wave + i * LPH, cbase, clo, chi, rb);

				f32x4 sc[NT];
#pragma unroll
				for (int t = 0; t < NT; ++t)
				{
					if constexpr (PACK)
					{
						f32x4 s = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
						for (int kk = 0; kk < KK; ++kk) s = mfma16x16x32(as_bf16x8(X.k[t][kk]), qhi[kk], s);
						// column c + G (lane + G of the 16-lane row) holds the lo sum
#pragma unroll
						for (int e = 0; e < 4; ++e)
							s[e] = s[e] + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s[e]), 0x100 + G, 0xf,
							                                                         0xf, false));
						sc[t] = s;
					}
					else
						sc[t] = scores_hilo<KK>(X.k[t], qhi, qlo);
				}
				const bool reload = i + DEPTH < n_wchunks; // uniform
				if (reload) load_k(X, i + DEPTH);

				// This chunk's V rows into the wavefront's LDS tile, then the
				// loads of chunk i + DEPTH into the freed registers.
#pragma unroll
				for (int j = 0; j < NV; ++j)
					*reinterpret_cast<u32x4*>(vt + (j * KPL + lane / LPK) * VPITCH + 8 * (lane % LPK)) = X.v[j];
				if (reload) load_v(X, i + DEPTH);

				// Online softmax per head (column), with a lazy offset.
				float m_loc = softmax_mask_max<NT>(sc, cbase, col_s0, col_s1, col_real, CH);
				const float m_new = lazy_offset(m_run, m_loc);
				const float m_use = m_new == -INFINITY ? 0.0f : m_new;
				const float alpha = m_new == m_run ? 1.0f : fast_exp2(m_run - m_use);
				const bool rescale = __builtin_amdgcn_ballot_w64(col_real && m_new != m_run) != 0; // uniform
				m_run = m_new;
				float lsum = 0.0f;
				u32x4 pb[NC][2];
#pragma unroll
				for (int c = 0; c < NC; ++c)
				{
					float w[8];
#pragma unroll
					for (int e = 0; e < 4; ++e)
					{
						w[e] = fast_exp2(sc[2 * c][e] - m_use);
						w[4 + e] = fast_exp2(sc[2 * c + 1][e] - m_use);
					}
					p_operand(w, pb[c], lsum);
				}
				l_run = l_run * alpha + lsum;
				if (rescale)
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
						pv_mfma(acc_o[db], u32x4{lo.x, lo.y, hi.x, hi.y}, pb[c]);
					}
				wave_sync(); // V is read before the next chunk overwrites it
			};
			int i = 0;
			if constexpr (DEPTH == 2)
				for (; i + 1 < n_wchunks; i += 2)
				{
					chunk(X0, i);
					chunk(X1, i + 1);
				}
			for (; i < n_wchunks; ++i) chunk(X0, i);

			// Wavefront partial: each (head, d) of O^T has one owner lane.
			l_run += __shfl_xor(l_run, 16);
			l_run += __shfl_xor(l_run, 32);
			if (tt < n_tt) // col < n_tt * G <= T * G
			{
#pragma unroll
				for (int db = 0; db < DB; ++db) *reinterpret_cast<f32x4*>(&s_wpart[wave][col][16 * db + 4 * grp]) = acc_o[db];
				if (grp == 0)
				{
					s_wpart[wave][col][HD] = m_run;
					s_wpart[wave][col][HD + 1] = l_run;
				}
			}
			__syncthreads();
			write_wg_result<HD, G, W, HPW>(p, &s_wpart[0][0][0], T * G * PW, tok0, n_tt * G, split, hg);
		}

		// The BF16 kernel for a session batch: NTL tiles of 16 MFMA columns,
		// 16 * NTL / G tokens per work-group, so a 16-token batch streams each
		// K and V row once. Q (hi and lo) sits in LDS; per chunk the scores of
		// every tile come from the same K registers and the V^T tile is read
		// back once per tile. Each column goes through exactly the operations
		// of decode_bf16_kernel (same products, same order), so a token gets
		// the bits of its one-token call here too.
		template <int HD, int G, int W, int CHK, int NTL, int HPW>
		__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(1, 1))) void decode_bf16_multi_kernel(
			const decode_params p)
		{
			using S = bf16_shape<HD, CHK>;
			constexpr int CH = S::CH, NT = S::NT, NC = S::NC, KK = S::KK, DB = S::DB, LPK = S::LPK, KPL = S::KPL,
			              NV = S::NV, VPITCH = S::VPITCH;
			constexpr int PW = part_pitch<HD>(), T = 16 * NTL / G, LPH = W / HPW;
			static_assert(NTL >= 2 && (16 * NTL) % G == 0, "tiles per work-group");

			// Each wavefront's partials go into its own V tile after its last chunk.
			__shared__ __attribute__((aligned(16))) uint16_t s_v[W][CH * VPITCH];
			__shared__ __attribute__((aligned(16))) u32x4 s_q[HPW][NTL][KK][2][64]; // B operands, hi and lo, per head
			static_assert(16 * PW * 4 <= CH * VPITCH * 2, "partials fit a V tile");
			constexpr int kTileFloats = CH * VPITCH / 2;

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
			const int col = lane & 15;
			const int grp = lane >> 4;
			const int hh = wave % HPW, hlane = wave / HPW; // this wavefront's head in the work-group, its lane
			const int n_hg = p.n_kv / HPW, n_zg = (p.n_tok + T - 1) / T;
			int hg, split, zg;
			wg_coords(blockIdx.x, p.n_split, n_hg, n_zg, hg, split, zg);
			const int kvh = head_of<HPW>(hg, hh, p.n_kv);
			const int tok0 = zg * T;
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
			int c_wave = c_first + ((hlane - c_first % LPH) + LPH) % LPH;
			const bool has_chunk = c_wave <= c_last;
			const int n_wchunks = has_chunk ? (c_last - c_wave) / LPH + 1 : 0;
			const int c_wlast = c_wave + (n_wchunks - 1) * LPH;

			u32x4 kreg[NT][KK];
			u32x4 vreg[NV];
			auto chunk_bounds = [&](int c, int& cbase, int& clo, int& chi, int& rb) __attribute__((always_inline))
			{
				cbase = sbase + c * CH;
				clo = max(s0, cbase);
				chi = min(s1, cbase + CH - 1);
				rb = clo % p.rows; // (a select here costs this kernel registers it does not have)
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

			// Q^T of every tile of each head into LDS as the B operands, scaled
			// into log2 units and split into bf16 hi + lo (entry (head, tl, kk, l)
			// is lane l's 8 elements 32 kk + 8 (l / 16) .. of column 16 tl + l % 16).
			// A wavefront load covers elements 32 kk .. 32 kk + 31 of 8 columns
			// (whole 128-byte lines), 16 bytes per lane; each thread converts
			// its 4 elements and writes their 8 bytes of each half. Every Q load
			// goes out first, then the first chunk's K and V rows, so the
			// conversion waits for Q alone (loads complete in order) and nothing
			// waits for a round trip per entry.
			constexpr int kQCols = HPW * 16 * NTL; // (head, column) pairs
			constexpr int kQLoads = kQCols * HD / 4 / (64 * W);
			static_assert(kQLoads * 64 * W * 4 == kQCols * HD && kQCols % 8 == 0, "Q float4s per thread");
			// float4 f: element 4 (f % 8) of block kk = (f / 64) % KK, column
			// 8 ((f / 64) / KK) + (f / 8) % 8 of the (head, column) pairs.
			auto q_item = [&](int u, int& qh, int& gc, int& kk, int& j) __attribute__((always_inline))
			{
				const int f = static_cast<int>(threadIdx.x) + u * 64 * W;
				j = f & 7;
				kk = (f >> 6) % KK;
				const int r = 8 * ((f >> 6) / KK) + ((f >> 3) & 7);
				qh = r / (16 * NTL);
				gc = r % (16 * NTL);
			};
			float4 qv[kQLoads];
#pragma unroll
			for (int u = 0; u < kQLoads; ++u)
			{
				int qh, gc, kk, j;
				q_item(u, qh, gc, kk, j);
				const int tt = gc / G;
				// (a column past the batch reads its group's first token and is zeroed below)
				const float* qp = p.q +
				                  (static_cast<size_t>(tok0 + (tt < n_tt ? tt : 0)) * p.n_head +
				                   head_of<HPW>(hg, qh, p.n_kv) * G + gc % G) * HD +
				                  32 * kk + 4 * j;
				qv[u] = *reinterpret_cast<const float4*>(qp);
			}
			if (has_chunk)
			{
				load_k(c_wave);
				load_v(c_wave);
			}
#pragma unroll
			for (int u = 0; u < kQLoads; ++u)
			{
				int qh, gc, kk, j;
				q_item(u, qh, gc, kk, j);
				const bool real = gc / G < n_tt;
				const float4 x = make_float4(real ? qv[u].x * p.qscale : 0.0f, real ? qv[u].y * p.qscale : 0.0f,
				                             real ? qv[u].z * p.qscale : 0.0f, real ? qv[u].w * p.qscale : 0.0f);
				u32x2 hi, lo;
				split_bf16x4(x, hi, lo);
				const int l = (gc & 15) + 16 * (j >> 1), tl = gc >> 4;
				reinterpret_cast<u32x2*>(&s_q[qh][tl][kk][0][l])[j & 1] = hi;
				reinterpret_cast<u32x2*>(&s_q[qh][tl][kk][1][l])[j & 1] = lo;
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
				// This chunk's V rows (loaded through the previous chunk) into the
				// wavefront's V^T tile first, so their registers are free for the
				// scores.
#pragma unroll
				for (int j = 0; j < NV; ++j)
					*reinterpret_cast<u32x4*>(vt + (j * KPL + lane / LPK) * VPITCH + 8 * (lane % LPK)) = vreg[j];
				wave_sync();
				// V^T read back once for all tiles (the A operands of P.V).
				u32x4 vta[NC][DB];
#pragma unroll
				for (int c = 0; c < NC; ++c)
#pragma unroll
					for (int db = 0; db < DB; ++db)
					{
						const uint16_t* r0 = vt + (32 * c + 4 * grp + (col >> 2)) * VPITCH + 16 * db + 4 * (col & 3);
						const u32x2 lo = vt_read(r0);
						const u32x2 hi = vt_read(r0 + 16 * VPITCH);
						vta[c][db] = u32x4{lo.x, lo.y, hi.x, hi.y};
					}

				// A tile's scores (the hi and lo products in their own chains,
				// added once: the operations of scores_hilo), then its softmax and
				// P.V. The last two tiles' scores come first, then the next chunk's
				// K rows load (two tiles of work to land in), and its V rows before
				// the last tile's softmax (all four tiles' scores at once, or the V
				// rows a tile earlier, would not fit the registers).
				auto tile_scores = [&](int tl, f32x4 (&out)[NT]) __attribute__((always_inline))
				{
					// (the lo chain accumulates in sc, the hi chain in sh)
					f32x4 sc[NT], sh[NT];
#pragma unroll
					for (int t = 0; t < NT; ++t) sh[t] = sc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
					for (int kk = 0; kk < KK; ++kk)
					{
						const bf16x8 qh = __builtin_bit_cast(bf16x8, s_q[hh][tl][kk][0][lane]);
						const bf16x8 ql = __builtin_bit_cast(bf16x8, s_q[hh][tl][kk][1][lane]);
#pragma unroll
						for (int t = 0; t < NT; ++t)
						{
							const bf16x8 a = as_bf16x8(kreg[t][kk]);
							sh[t] = mfma16x16x32(a, qh, sh[t]);
							sc[t] = mfma16x16x32(a, ql, sc[t]);
						}
					}
#pragma unroll
					for (int t = 0; t < NT; ++t) out[t] = sh[t] + sc[t];
				};
				auto tile_softmax_pv = [&](int tl, f32x4 (&sc)[NT]) __attribute__((always_inline))
				{
					const bool real = (16 * tl + col) / G < n_tt;
					const float m_loc = softmax_mask_max<NT>(sc, cbase, col_s0[tl], col_s1[tl], real, CH);
					const float m_new = lazy_offset(m_run[tl], m_loc);
					const float m_use = m_new == -INFINITY ? 0.0f : m_new;
					const float alpha = m_new == m_run[tl] ? 1.0f : fast_exp2(m_run[tl] - m_use);
					const bool rescale = __builtin_amdgcn_ballot_w64(real && m_new != m_run[tl]) != 0; // uniform
					m_run[tl] = m_new;
					float lsum = 0.0f;
					u32x4 pb[NC][2];
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
						p_operand(w, pb[c], lsum);
					}
					l_run[tl] = l_run[tl] * alpha + lsum;
					if (rescale)
#pragma unroll
						for (int db = 0; db < DB; ++db) acc_o[tl][db] *= alpha;
#pragma unroll
					for (int c = 0; c < NC; ++c)
#pragma unroll
						for (int db = 0; db < DB; ++db) pv_mfma(acc_o[tl][db], vta[c][db], pb[c]);
				};
#pragma unroll
				for (int tl = 0; tl < NTL - 2; ++tl)
				{
					f32x4 sc[NT];
					tile_scores(tl, sc);
					tile_softmax_pv(tl, sc);
				}
				f32x4 sa[NT], sb[NT];
				tile_scores(NTL - 2, sa);
				tile_scores(NTL - 1, sb);
				load_k(cw + LPH);
				tile_softmax_pv(NTL - 2, sa);
				load_v(cw + LPH);
				tile_softmax_pv(NTL - 1, sb);
				wave_sync(); // V is read before the next chunk overwrites it
			};
			for (int i = 0; i < n_wchunks; ++i, c_wave += LPH) chunk(c_wave);

			// One tile at a time through the wavefront merge; a wavefront's
			// partials go into its own V tile (read by it only until here).
			float* s_wpart = reinterpret_cast<float*>(&s_v[0][0]);
			float* wpart = s_wpart + wave * kTileFloats;
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
					for (int db = 0; db < DB; ++db) *reinterpret_cast<f32x4*>(&wpart[col * PW + 16 * db + 4 * grp]) = acc_o[tl][db];
					if (grp == 0)
					{
						wpart[col * PW + HD] = m_run[tl];
						wpart[col * PW + HD + 1] = lr;
					}
				}
				__syncthreads();
				if (n_cols > 0)
					write_wg_result<HD, G, W, HPW, false>(p, s_wpart, kTileFloats, tok0 + 16 * tl / G, n_cols, split, hg);
				__syncthreads(); // the partials are read before the next tile overwrites them
			}
		}


		// Keys per wavefront chunk of the BF16 kernel (4 wavefronts, one per
		// SIMD). Measured at 32k keys: 8 wavefronts of 32-key chunks (two per
		// SIMD) run 2% slower.
		constexpr int bf16_chunk(int head_dim) { return head_dim == 256 ? 32 : 64; }


		template <int HD, int G, bool BF16>
		void launch_g(const decode_params& p, int n_tok, hipStream_t stream)
		{
			if constexpr (BF16)
			{
				// One token: the one-token instance (less LDS for partials);
				// batches: 16 / G tokens per work-group, or four tiles of them.
				// All compute a token's column with the same operations.
				constexpr int T = 16 / G, TM = 64 / G; // tokens per work-group: one tile, four tiles
				auto go = [&](auto hpw_tag)
				{
					constexpr int HPW = decltype(hpw_tag)::value;
					const int n_hg = p.n_kv / HPW;
					if (n_tok == 1)
						decode_bf16_kernel<HD, G, 4, bf16_chunk(HD), 1, HPW><<<dim3(n_hg, p.n_split), 256, 0, stream>>>(p);
					else
					{
						bool multi = false;
						if constexpr (HD <= 128) // (at head_dim 256 four tiles do not fit the registers)
						{
							if (n_tok > T)
							{
								multi = true;
								decode_bf16_multi_kernel<HD, G, 4, bf16_chunk(HD), 4, HPW>
									<<<p.n_split * n_hg * ((n_tok + TM - 1) / TM), 256, 0, stream>>>(p);
							}
						}
						if (!multi)
							decode_bf16_kernel<HD, G, 4, bf16_chunk(HD), T, HPW>
								<<<p.n_split * n_hg * ((n_tok + T - 1) / T), 256, 0, stream>>>(p);
					}
				};
				if (bf16_heads_per_wg(p.n_kv) == 2)
					go(std::integral_constant<int, 2>{});
				else
					go(std::integral_constant<int, 1>{});
			}
			else
				f32_decode_kernel<HD, G><<<dim3(p.n_split, p.n_kv, n_tok), 256, 0, stream>>>(p);
			// The merge: a quarter head per work-group while that makes at most
			// 256 work-groups, else whole heads.
			if (fused_merge_on(p))
				return;
			if (p.n_split > 1 && p.n_kv * G * n_tok <= 64)
				launch_merge<HD, G, 4>(p, n_tok, stream);
			else if (p.n_split > 1)
				launch_merge<HD, G, 1>(p, n_tok, stream);
		}

		template <int HD, bool BF16>
		bool launch_hd(const decode_params& p, int n_tok, int group, hipStream_t stream)
		{
			switch (group)
			{
			case 1: launch_g<HD, 1, BF16>(p, n_tok, stream); return true;
			case 2: launch_g<HD, 2, BF16>(p, n_tok, stream); return true;
			case 4: launch_g<HD, 4, BF16>(p, n_tok, stream); return true;
			case 8: launch_g<HD, 8, BF16>(p, n_tok, stream); return true;
			default: return false;
			}
		}
	}

	int decode_wg_keys(int head_dim, int group, bool bf16, int n_kv)
	{
		if (!mfma_shape(head_dim, group)) return 256;
		const int lanes = bf16 ? 4 / bf16_heads_per_wg(n_kv) : 4; // wavefronts per KV head
		switch (head_dim)
		{
		case 64: return lanes * (bf16 ? bf16_chunk(64) : f32_shape<64>::CH);
		case 128: return lanes * (bf16 ? bf16_chunk(128) : f32_shape<128>::CH);
		case 256: return lanes * (bf16 ? bf16_chunk(256) : f32_shape<256>::CH);
		default: return 0;
		}
	}

	int decode_chunk_keys(int head_dim, int group, bool bf16)
	{
		if (!mfma_shape(head_dim, group)) return 256;
		switch (head_dim)
		{
		case 64: return bf16 ? bf16_chunk(64) : f32_shape<64>::CH;
		case 128: return bf16 ? bf16_chunk(128) : f32_shape<128>::CH;
		case 256: return bf16 ? bf16_chunk(256) : f32_shape<256>::CH;
		default: return 0;
		}
	}

	int decode_groups(int n_kv, bool bf16, int head_dim, int group)
	{
		return bf16 && mfma_shape(head_dim, group) ? n_kv / bf16_heads_per_wg(n_kv) : n_kv;
	}

	bool launch_decode(const decode_params& p, int n_tok, int head_dim, int group, bool bf16, hipStream_t stream)
	{
		if (!mfma_shape(head_dim, group)) return launch_decode_generic(p, n_tok, head_dim, group, bf16, stream);
		switch (head_dim)
		{
		case 64:
			return bf16 ? launch_hd<64, true>(p, n_tok, group, stream) : launch_hd<64, false>(p, n_tok, group, stream);
		case 128:
			return bf16 ? launch_hd<128, true>(p, n_tok, group, stream) : launch_hd<128, false>(p, n_tok, group, stream);
		case 256:
			return bf16 ? launch_hd<256, true>(p, n_tok, group, stream) : launch_hd<256, false>(p, n_tok, group, stream);
		default: return false;
		}
	}
}
