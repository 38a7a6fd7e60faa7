// Flash attention on CDNA4 MFMA for a batch of query tokens (nnc's batch
// path, reference src/libnnc/model.cpp:1750-1757, and the chunked prefill of
// a long prompt), BF16 K/V.
//
// Rows of the problem are (token, query head) pairs of one KV head, token
// major, so the heads of a GQA group sit in adjacent rows and share every key
// the work-group reads. Grid: n_kv * n_qtiles work-groups. A work-group owns
// RG row groups of 32 rows (RG = 2 at head_dim 64 and 128: 64 rows, eight
// wavefronts, one work-group per CU; head_dim 256 runs prefill16_kernel
// below, two row groups of 16 rows) and walks its key range in steps of 128
// keys. Wavefront
// (g, r) takes keys 32 g .. 32 g + 31 of each step for the 32 rows of row
// group r, so every product is one 32 x 32 tile (v_mfma_f32_32x32x16, which
// one wavefront keeps near the matrix peak); the row groups share each key
// group's K and V tiles, which halves the bytes loaded per product. Each
// wavefront keeps its own online softmax, and the four key groups of a row
// group merge once, in LDS, at the end.
//
// The work-group first stages its Q rows through LDS (whole rows per
// wavefront load, pre-scaled into log2 units and split into bf16 hi + lo, so
// two MFMAs against the exact bf16 K give near-fp32 scores); every
// wavefront then keeps both halves of its B operand in registers (at
// head_dim 256 it reads them from LDS). V comes from one of two copies:
//   - an fp16 copy (exact copies of the bf16 values, kept beside the cache
//     and used while every value in it is within +-8, kF16CopyMax, where
//     P's rounding moves an output by at most 2^-11 * 8): P goes in fp16
//     rounded to nearest, one MFMA per product;
//   - the bf16 V itself (no copy, or a larger value in it): P is split into
//     bf16 hi + lo, two MFMAs per product, near-fp32.
// Per step, a key group's 32 K rows and 32 V rows arrive in its LDS tiles
// by LDS-DMA (buffer_load ... lds, 16 bytes per lane, rows XOR-swizzled in
// 16-byte slots so the reads below are conflict-free; the fp16 copy's tile
// is one 32-row group of its blocked layout, f16_copy_index, as it lies),
// issued during the previous step (RG = 2: two stages, the DMAs split
// between the row groups, one barrier per step; RG = 1: each wavefront's
// own tiles, one stage). With the copy the walk starts at the key range's
// first key rounded down to 32, so every tile is a whole group:
//   S^T = K . Q^T      v_mfma_f32_32x32x16, K rows as the A operand and Q^T
//                      as B. The accumulator starts at -m (the row's running
//                      offset), so the scores come out already shifted.
//                      Meanwhile V^T is read into registers: from the
//                      copy's blocks with plain 16-byte reads, from the bf16
//                      V transposed (ds_read_b64_tr_b16);
//   softmax            in fp32 and log2 units, weights exp2(s - m) with the
//                      row's offset m set 8 below its largest score so far:
//                      m is raised only when a score passes it by more than
//                      15, so weights stay in (0, 2^15] (fp16's range) and the
//                      O rescale is rare, and the row sum is at least 2^8, so
//                      fp16's subnormal steps (2^-24) are negligible in it; the
//                      two halves of a row's 32 scores meet through
//                      v_permlane32_swap;
//   O^T += V^T . P^T   P as the B operand straight from the score registers
//                      (key order permuted to match). In fp16 the row sums l
//                      come from the same rounded P through v_dot2_f32_f16, so
//                      numerator and denominator see identical weights; in
//                      bf16 they are fp32 sums of the unrounded weights.
// K/V are read through buffer descriptors whose range check returns zeros
// for rows past the key range without touching memory; a range that wraps a
// ring buffer is walked as two contiguous segments. Masking is applied only
// to steps that cross some row's span edge or a segment's end (masked keys
// weigh exactly 0). The final merge sums the wavefronts in a fixed order, so
// results are the same run to run.
#include "device_common.h"
#include "kernels.h"

#include <type_traits>



namespace nnchip
{
	namespace
	{
		constexpr int kKG = 4; // key groups: the key quarters of a step
		constexpr int kWK = 32; // keys per wavefront per step (one MFMA tile)
		constexpr int kStep = kKG * kWK; // keys per work-group step
		constexpr float kBias = 8.0f; // a raised offset sits this far below the row's max (log2 units)
		constexpr float kLazy = 15.0f; // max growth of a row's scores over its offset (weights up to 2^15)
		constexpr int kBufferFlags = 0x00020000; // buffer descriptor word 3: raw 32-bit data

		// A work-group is RG row groups of 32 rows times kKG key groups, one
		// wavefront each; the row groups of a key group share its K and V
		// tiles. LDS: the K and V tiles (RG = 2: two stages, double-buffered),
		// Q's lo half, Q's hi half (staged once); the merge buffer reuses the
		// tiles and Q, and the merge's row statistics sit at kStats. RG = 1 at
		// head_dim 128 is 80 KiB, so two work-groups (two wavefronts per SIMD)
		// share a CU; RG = 2 is 160 KiB, one work-group of eight wavefronts.
		template <int HD, int RG>
		struct prefill_shape
		{
			static constexpr int WAVES = kKG * RG;
			static constexpr int ROWS = 32 * RG; // rows per work-group
			static constexpr int STAGES = RG == 1 ? 1 : 2;
			// wavefronts per SIMD: HD == 256 ? 1 : 2 (in the kernel's attributes)
			// Q's B operand (hi and lo halves) held in registers; at head_dim 256
			// it would not fit beside the accumulators, and is read from LDS.
			static constexpr bool QREG = HD != 256;
			static constexpr int KT = HD / 16; // QK MFMAs per Q half (16 elements of d each)
			static constexpr int DBK = HD / 32; // 32-row d blocks of O^T
			static constexpr int LPK = HD / 8; // lanes per tile row (16 bytes each)
			static constexpr int KPL = 64 / LPK; // tile rows per DMA
			static constexpr int NV = kWK / KPL; // DMAs per tile per step
			static constexpr int OPITCH = HD + 4; // floats per row in the final merge
			static constexpr int kTile = kWK * HD * 2; // bytes of one K (or V) tile
			static constexpr int kStage = kKG * 2 * kTile; // the tiles of one step
			static constexpr int kTiles = STAGES * kStage;
			static constexpr int kQ = ROWS * HD * 2; // bytes of one bf16 half of Q
			static constexpr int kQlo = kTiles; // offsets
			static constexpr int kQhi = kTiles + kQ;
			static constexpr int kLds = kTiles + 2 * kQ;
			static constexpr int kStatBytes = 2 * WAVES * 32 * 4;
			static constexpr int kStats = RG == 1 ? kQhi : kLds - kStatBytes;
			static constexpr int kOBytes = WAVES * 32 * OPITCH * 4;
			static_assert(NV >= 1 && KPL * NV == kWK && NV % RG == 0, "unsupported prefill shape");
			static_assert(kOBytes <= kStats && kStats + kStatBytes <= kLds, "merge buffer layout");
			static_assert(kLds <= 160 * 1024, "prefill LDS budget");
			static_assert(RG == 1 || QREG, "two row groups need Q in registers (the Q region is reused)");
		};

		// Two 16-bit halves of one row of O^T's A operand: lane (g, c) of the
		// ds_read_b64_tr_b16 gives T[row0 + 4g + k][d0 + c], k = 0..3, when lane
		// c of each 16-lane group points at T[row0 + 4g + c / 4][d0 + 4 (c % 4)].
		__device__ __forceinline__ u32x2 tr_read(const uint16_t* row_ptr)
		{
			typedef short s16x4 __attribute__((ext_vector_type(4)));
			typedef __attribute__((address_space(3))) s16x4* lds_s16x4;
			const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(row_ptr));
			return __builtin_bit_cast(u32x2, v);
		}

		// 16-byte slot swizzle of row `row` of a V tile, in whole 64-byte
		// groups: a half-wavefront's transposing reads cover one 64-byte
		// segment of each of four consecutive rows, which land in distinct
		// banks.
		template <int HD>
		__device__ __forceinline__ int vswz(int row)
		{
			return HD == 64 ? 4 * ((row >> 1) & 1) : 4 * (row & 3);
		}

		// 16-byte slot swizzle of row `row` of a K tile: the A-operand reads of
		// 16 consecutive rows at one slot land in distinct banks.
		template <int HD>
		__device__ __forceinline__ int kswz(int row)
		{
			return HD == 64 ? (row >> 1) & 7 : row & 15;
		}

		// DMA j of a tile: 16 bytes per lane from buffer offset voffset into
		// the tile at byte 1024 j + 16 l. The instruction offset (1024 (j % 4))
		// is added to both the buffer offset (and its range check) and the LDS
		// address, so DMAs j = 4 g .. 4 g + 3 share the LDS base tile + 4096 g:
		// one M0 value for four DMAs. voffset >= 1024 j always holds for the
		// tiles here (row r of DMA j starts at r * row_bytes >= 1024 j).
		__device__ __forceinline__ void load_lds16_grouped(__amdgpu_buffer_rsrc_t rsrc, uint16_t* tile, int j,
		                                                   uint32_t voffset)
		{
			typedef __attribute__((address_space(3))) void* lds_ptr;
			const lds_ptr base = (lds_ptr)(reinterpret_cast<char*>(tile) + 4096 * (j >> 2));
			switch (j & 3) // j is a constant after unrolling; the offset must be an immediate
			{
			case 0: __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, base, 16, voffset, 0, 0, 0); break;
			case 1: __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, base, 16, voffset - 1024u, 0, 1024, 0); break;
			case 2: __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, base, 16, voffset - 2048u, 0, 2048, 0); break;
			default: __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, base, 16, voffset - 3072u, 0, 3072, 0); break;
			}
		}

		// Waits until every LDS access this wavefront issued has completed
		// (s_waitcnt lgkmcnt(0); the vector-memory and export counters at
		// their maximum, i.e. not waited on: gfx9 encoding vmcnt[3:0] = 0xf,
		// expcnt[6:4] = 7, lgkmcnt[11:8] = 0, vmcnt[15:14] = 3). Nothing is
		// scheduled across it.
		__device__ __forceinline__ void lds_reads_done()
		{
			__builtin_amdgcn_sched_barrier(0);
			__builtin_amdgcn_s_waitcnt(0xC07F);
			__builtin_amdgcn_sched_barrier(0);
		}

		// Waits until this wavefront's LDS-DMA loads have landed (s_waitcnt
		// vmcnt(0); expcnt and lgkmcnt at their maximum, i.e. not waited on:
		// gfx9 encoding vmcnt[3:0] = 0, expcnt[6:4] = 7, lgkmcnt[11:8] = 0xf,
		// vmcnt[15:14] = 0). The compiler's own tracking of LDS-DMA writes
		// does not reliably order later LDS reads of the same tile after them,
		// so every step waits explicitly. Nothing is scheduled across it.
		__device__ __forceinline__ void dma_done()
		{
			__builtin_amdgcn_sched_barrier(0);
			__builtin_amdgcn_s_waitcnt(0x0F70);
			__builtin_amdgcn_sched_barrier(0);
		}

		// Q rows row0 .. row0 + ROWS - 1 of KV head kvh (row r: token r / G,
		// query head kvh * G + r % G), pre-scaled into log2 units and split
		// into bf16 hi + lo, into LDS in the K tiles' layout (row r, 16-byte
		// slot s at s ^ kswz(r)); rows from n_rows on are zero. Thread t
		// loads float4s t, t + NTHR, ... of the rows taken in order, so one
		// wavefront load covers whole rows (a token's G query heads are
		// adjacent in memory: whole cache lines, contiguous runs), and writes
		// the 8 bytes of each half that its float4 gives. All loads go out
		// before the first conversion.
		template <int HD, int G, int ROWS, int NTHR>
		__device__ __forceinline__ void stage_q(const float* q, size_t q_stride, float qscale, int kvh, int row0,
		                                        int n_rows, uint16_t* s_qhi, uint16_t* s_qlo)
		{
			constexpr int F4 = HD / 4, N = ROWS * F4 / NTHR;
			static_assert(N * NTHR == ROWS * F4, "Q float4s per thread");
			float4 a[N];
#pragma unroll
			for (int u = 0; u < N; ++u)
			{
				const int f = u * NTHR + static_cast<int>(threadIdx.x), grow = row0 + f / F4;
				a[u] = grow < n_rows ? *reinterpret_cast<const float4*>(
										   q + static_cast<size_t>(grow / G) * q_stride +
										   static_cast<size_t>(kvh * G + grow % G) * HD + 4 * (f % F4))
				                     : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
			}
#pragma unroll
			for (int u = 0; u < N; ++u)
			{
				const int f = u * NTHR + static_cast<int>(threadIdx.x), r = f / F4, c4 = f % F4;
				u32x2 hi, lo;
				split_bf16x4(make_float4(a[u].x * qscale, a[u].y * qscale, a[u].z * qscale, a[u].w * qscale), hi, lo);
				const int off = r * HD + 8 * ((c4 >> 1) ^ kswz<HD>(r)) + 4 * (c4 & 1);
				*reinterpret_cast<u32x2*>(s_qhi + off) = hi;
				*reinterpret_cast<u32x2*>(s_qlo + off) = lo;
			}
		}

		template <int HD, int G, int RG>
		__global__ __launch_bounds__(64 * kKG * RG)
			__attribute__((amdgpu_waves_per_eu(HD == 256 ? 1 : 2, HD == 256 ? 1 : 2))) void prefill_kernel(
				const prefill_params p)
		{
			using S = prefill_shape<HD, RG>;
			constexpr int KT = S::KT, DBK = S::DBK, LPK = S::LPK, KPL = S::KPL, NV = S::NV, OPITCH = S::OPITCH;
			constexpr int kWaves = S::WAVES, kRows = S::ROWS;

			__shared__ __attribute__((aligned(16))) unsigned char s_raw[S::kLds];

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: keeps step control scalar
			const int kg = wave % kKG, rg = wave / kKG; // this wavefront's key group and row group
			const int r32 = lane & 31; // this lane's row of the tile (and key, as an A-operand row)
			const int h = lane >> 5; // which half of an MFMA's k range this lane holds

			// Work-groups of one KV head run on one XCD (blockIdx.x % 8 picks
			// the XCD), so its K/V rows are shared through that XCD's L2. Within
			// a head the first half of the work-groups take the query tiles with
			// the most keys, heaviest first, and the second half the lightest
			// first, so the two that share a CU carry about equal work.
			int bid = blockIdx.x;
			const int n_wg = gridDim.x;
			if ((n_wg & 7) == 0) bid = (bid & 7) * (n_wg >> 3) + (bid >> 3);
			const int kvh = bid / p.n_qtiles;
			const int j = bid % p.n_qtiles, half = (p.n_qtiles + 1) / 2;
			const int qt = j < half ? p.n_qtiles - 1 - j : j - half;

			const int n_rows = p.n_tok * G;
			const int row0 = qt * kRows;
			const size_t q_stride = static_cast<size_t>(p.n_head) * HD;

			// The work-group's key range [kmin, kmax], and [first_hi, last_lo],
			// the keys every one of its rows sees (span ends grow with the
			// position).
			int kmin, kmax, first_hi, last_lo;
			{
				const int t0 = row0 / G, t1 = min(p.n_tok - 1, (row0 + kRows - 1) / G);
				attn_span(p.causal, p.window, p.pos0 + t0, p.n_seq, kmin, last_lo);
				attn_span(p.causal, p.window, p.pos0 + t1, p.n_seq, first_hi, kmax);
			}
			// This lane's row and its span.
			const int my_row = row0 + 32 * rg + r32;
			int rfirst = 1, rlast = 0; // no key
			if (my_row < n_rows) attn_span(p.causal, p.window, p.pos0 + my_row / G, p.n_seq, rfirst, rlast);

			// V's fp16 copy when the buffer has one and every value now in it
			// is within the copy's limit (and, in a buffer whose rows are not a
			// whole number of the copy's 32-row groups, the range does not
			// wrap); else the bf16 V itself. The copy's tiles are whole groups,
			// so with it the walk starts at kmin rounded down to 32 (the keys
			// before kmin are masked like any outside a row's span).
			const bool use16 = p.V16 != nullptr && __builtin_amdgcn_readfirstlane(*p.n_bad) == 0 &&
			                   ((p.rows & 31) == 0 || kmax < p.rows);
			const int kbeg = use16 ? kmin & ~31 : kmin;

			// The key range as contiguous segments of rows: keys kbeg .. from row
			// rb0 up to the buffer's end, then (a ring that wraps) the rest from
			// row 0. The host guarantees the range is shorter than the buffer
			// (kmin .. kmax; the keys before kmin may alias rows of the last
			// ones, and are masked).
			const int span = kmax >= kmin ? kmax - kbeg + 1 : 0;
			const int rb0 = span > 0 ? kbeg % p.rows : 0;
			const int len1 = min(span, p.rows - rb0);
			const int len2 = span - len1;
			const int n1 = (len1 + kStep - 1) / kStep;
			const int n_steps = n1 + (len2 + kStep - 1) / kStep;
			const int wrap_key = kbeg + len1; // segment 2's first key

			// Byte offsets are 32-bit (the host keeps a buffer under 2 GiB).
			const uint32_t row_bytes = static_cast<uint32_t>(p.kv_dim) * 2;
			const uint32_t head_bytes = static_cast<uint32_t>(kvh) * HD * 2;
			const char* kbase = static_cast<const char*>(p.K) + head_bytes;
			// (the copy's blocks hold 8 rows of each column: a head's columns
			// start 8 times as far in)
			const char* vbase = use16 ? static_cast<const char*>(p.V16) + 8 * head_bytes
			                          : static_cast<const char*>(p.V) + head_bytes;

			// Step i of the wavefront: its first key and the last key of its
			// segment; its descriptors are based at the block's first row and in
			// range up to the segment's last row (later rows read as zeros).
			auto step_key = [&](int i, int& seg_last) __attribute__((always_inline)) -> int
			{
				const bool second = i >= n1;
				seg_last = second ? kmax : wrap_key - 1;
				return (second ? wrap_key + (i - n1) * kStep : kbeg + i * kStep) + kg * kWK;
			};
			// In bytes from the buffer's start: the wavefront's block at step i
			// is at seg_off + i * step_bytes (seg_off per segment: the block of
			// step 0, or of step n1 moved back n1 steps), and the segment ends
			// at seg_end (its last row's head slice included). Everything stays
			// below 2^32 since a buffer is under 2 GiB.
			const uint32_t step_bytes = static_cast<uint32_t>(kStep) * row_bytes;
			const uint32_t seg1_off = static_cast<uint32_t>(rb0 + kg * kWK) * row_bytes;
			const uint32_t seg2_off = static_cast<uint32_t>(kg * kWK) * row_bytes - static_cast<uint32_t>(n1) * step_bytes;
			const uint32_t seg1_end = static_cast<uint32_t>(rb0 + len1 - 1) * row_bytes + HD * 2;
			const uint32_t seg2_end = static_cast<uint32_t>(kmax - wrap_key) * row_bytes + HD * 2; // used when len2 > 0
			// The same in the fp16 copy: a 32-row group takes the bytes of 32
			// rows, so a group starts where its first row would; a segment
			// ends with its last group's last block (rows past the segment in
			// that group are read and masked).
			auto group_end = [&](int last_row) __attribute__((always_inline)) -> uint32_t
			{
				return static_cast<uint32_t>(last_row >> 5) * 32 * row_bytes + 48 * row_bytes / 2 + 16 * HD;
			};
			const uint32_t v_seg1_end = use16 ? group_end(rb0 + len1 - 1) : seg1_end;
			const uint32_t v_seg2_end = use16 ? group_end(kmax - wrap_key) : seg2_end;
			auto step_rsrc = [&](int i, const char* base, bool is_v) __attribute__((always_inline))
			{
				const bool second = i >= n1;
				const uint32_t off = (second ? seg2_off : seg1_off) + static_cast<uint32_t>(i) * step_bytes;
				const uint32_t end = is_v ? (second ? v_seg2_end : v_seg1_end) : (second ? seg2_end : seg1_end);
				// (the clamp becomes a VALU saturating subtract: readfirstlane keeps
				// the descriptor in SGPRs)
				const uint32_t n = __builtin_amdgcn_readfirstlane(end > off ? end - off : 0u);
				return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base + off), 0, static_cast<int>(n),
				                                         kBufferFlags);
			};

			// Tile layout: DMA j fills tile rows j KPL .. + KPL, lane l the 16
			// bytes at l * 16, i.e. row j KPL + l / LPK, slot l % LPK, which holds
			// the row's 16-byte segment (l % LPK) ^ swizzle(row).
			// The row groups of a key group split its DMAs: row group rg issues
			// DMAs rg NV / RG .. of each tile.
			const int t_row = lane / LPK;
			auto k_tile = [&](int i) __attribute__((always_inline)) -> uint16_t*
			{
				return reinterpret_cast<uint16_t*>(s_raw + (S::STAGES == 2 ? (i & 1) : 0) * S::kStage) +
				       kg * 2 * kWK * HD;
			};
			// DMAs e0 .. e1 - 1 of this wavefront's 2 ND for step i: its K DMAs,
			// then its V DMAs (so a step's loads can be spread over the step).
			constexpr int ND = NV / RG;
			// In the fp16 copy, tile byte 1024 jj + 16 l (DMA jj) is byte w of
			// block b = jj / (HD / 64) (a block is 16 HD bytes), which lies
			// 16 kv_dim b + w past the group's start.
			static_assert(16 * HD % 1024 == 0, "the fp16 copy's blocks are whole DMAs");
			constexpr int DPB = 16 * HD / 1024; // DMAs per block of the copy
			auto load_part = [&](auto f16_tag, int i, int e0, int e1) __attribute__((always_inline))
			{
				constexpr bool F16 = decltype(f16_tag)::value;
				const __amdgpu_buffer_rsrc_t rk = step_rsrc(i, kbase, false);
				const __amdgpu_buffer_rsrc_t rv = step_rsrc(i, vbase, true);
				uint16_t* kt = k_tile(i);
				uint16_t* vt = kt + kWK * HD;
				// Each group of four DMAs shares one LDS base (the instruction
				// offset moves the LDS and buffer addresses alike), so the K tile,
				// then the V tile, needs one LDS base per 4 KiB.
#pragma unroll
				for (int e = e0; e < e1; ++e)
				{
					const bool is_v = e >= ND;
					const int jj = rg * ND + (is_v ? e - ND : e);
					const int row = jj * KPL + t_row;
					const uint32_t rb = static_cast<uint32_t>(row) * row_bytes;
					if (is_v && F16)
						load_lds16_grouped(rv, vt, jj, (jj / DPB) * 8 * row_bytes + 1024u * (jj % DPB) + 16u * lane);
					else if (is_v)
						load_lds16_grouped(rv, vt, jj, rb + 16u * static_cast<uint32_t>((lane % LPK) ^ vswz<HD>(row)));
					else
						load_lds16_grouped(rk, kt, jj, rb + 16u * static_cast<uint32_t>((lane % LPK) ^ kswz<HD>(row)));
				}
			};
			auto load_tiles = [&](auto f16_tag, int i) __attribute__((always_inline)) { load_part(f16_tag, i, 0, 2 * ND); };
			// The first step's tiles go out before Q is read, so the latencies overlap.
			if (n_steps > 0)
			{
				if (use16)
					load_tiles(std::true_type{}, 0);
				else
					load_tiles(std::false_type{}, 0);
			}

			// Q, pre-scaled into log2 units and split into bf16 hi + lo (two
			// MFMAs against the exact bf16 K give near-fp32 scores), in LDS in
			// the K tiles' layout.
			uint16_t* s_qlo = reinterpret_cast<uint16_t*>(s_raw + S::kQlo);
			uint16_t* s_qhi = reinterpret_cast<uint16_t*>(s_raw + S::kQhi);
			stage_q<HD, G, kRows, 64 * kWaves>(p.q, q_stride, p.qscale, kvh, row0, n_rows, s_qhi, s_qlo);
			__syncthreads();
			// Q^T as the B operand: lane l holds row l % 32, elements 16 t + 8 h .. + 8.
			auto q_slot = [&](int t) __attribute__((always_inline)) -> int
			{
				return r32 * HD + 8 * ((2 * t + h) ^ kswz<HD>(r32));
			};
			bf16x8 qhi[S::QREG ? KT : 1], qlo[S::QREG ? KT : 1];
			if constexpr (S::QREG)
			{
#pragma unroll
				for (int t = 0; t < KT; ++t)
				{
					qhi[t] = *reinterpret_cast<const bf16x8*>(s_qhi + 32 * rg * HD + q_slot(t));
					qlo[t] = *reinterpret_cast<const bf16x8*>(s_qlo + 32 * rg * HD + q_slot(t));
				}
			}

			f32x16 acc_o[DBK]; // O^T: lane l holds d = 32 b + 8 (i / 4) + 4 h + i % 4 of row l % 32
			float l_acc = 0.0f; // this lane's half of its row's sum of weights
			float m_off = -INFINITY; // the row's score offset (-inf until it has seen a key)
			f32x16 c_init; // S^T's accumulator start: -m_off, or 0 before the first key
#pragma unroll
			for (int b = 0; b < DBK; ++b)
#pragma unroll
				for (int e = 0; e < 16; ++e) acc_o[b][e] = 0.0f;
#pragma unroll
			for (int e = 0; e < 16; ++e) c_init[e] = 0.0f;
			// V^T read position of this lane: a 16-lane group q covers elements
			// 32 b + 16 (q & 1) .. + 16 of four tile rows 16 c + 4 h (+ 8).
			const int tq = (lane >> 4) & 1, ti = lane & 15;
			const f16x2 one2 = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};

			// V^T as read: lane (g, c) of a transposing read holds keys
			// 16 c' + 4 h + g .. of the tile rows below (both halves).
			auto vt_pair = [&](const uint16_t* vt, int c, int b) __attribute__((always_inline)) -> u32x4
			{
				const int slot = 4 * b + 2 * tq + ((ti & 3) >> 1), hf = 4 * (ti & 1);
				const int ra = 16 * c + 4 * h + (ti >> 2), rb = ra + 8;
				const u32x2 lo = tr_read(vt + ra * HD + 8 * (slot ^ vswz<HD>(ra)) + hf);
				const u32x2 hi = tr_read(vt + rb * HD + 8 * (slot ^ vswz<HD>(rb)) + hf);
				return u32x4{lo.x, lo.y, hi.x, hi.y};
			};

			// S^T - m (32 keys x 32 rows) of step i, and its V^T read back: keys
			// 16 c + 4 h + j and 16 c + 8 + 4 h + j in k-slots j and 4 + j. A
			// wavefront in one of its MFMA phases raises its issue priority, so
			// the other wavefront of the SIMD fills the matrix core's shadow with
			// its softmax (measured: 4.6 % faster per prefill step).
			auto qk_phase = [&](auto f16_tag, int i, f32x16& sc, u32x4 (&vta)[2][DBK]) __attribute__((always_inline))
			{
				constexpr bool F16 = decltype(f16_tag)::value;
				const uint16_t* kt = k_tile(i);
				const uint16_t* vt = kt + kWK * HD;
				__builtin_amdgcn_s_setprio(1);
				sc = c_init;
				// bf16 K, Q as hi + lo: two MFMAs per 16 elements of d.
#pragma unroll
				for (int t = 0; t < KT; ++t)
				{
					const bf16x8 a = *reinterpret_cast<const bf16x8*>(kt + q_slot(t));
					if constexpr (S::QREG)
					{
						sc = mfma32x32x16(a, qhi[t], sc);
						sc = mfma32x32x16(a, qlo[t], sc);
					}
					else
					{
						sc = mfma32x32x16(a, *reinterpret_cast<const bf16x8*>(s_qhi + 32 * rg * HD + q_slot(t)), sc);
						sc = mfma32x32x16(a, *reinterpret_cast<const bf16x8*>(s_qlo + 32 * rg * HD + q_slot(t)), sc);
					}
				}
				// fp16 copy: block 2 c + h of the tile holds those eight keys of
				// every element, 16 bytes each: one plain read per operand.
#pragma unroll
				for (int c = 0; c < 2; ++c)
#pragma unroll
					for (int b = 0; b < DBK; ++b)
					{
						if constexpr (F16)
							vta[c][b] = *reinterpret_cast<const u32x4*>(vt + ((2 * c + h) * HD + 32 * b + r32) * 8);
						else
							vta[c][b] = vt_pair(vt, c, b);
					}
				__builtin_amdgcn_s_setprio(0);
			};

			// Masking, the online softmax and O^T += V^T . P^T of one step whose
			// scores and V^T are in registers.
			auto soft_phase = [&](auto f16_tag, int kw0, int seg_last, f32x16 sc, const u32x4 (&vta)[2][DBK])
				__attribute__((always_inline))
			{
				constexpr bool F16 = decltype(f16_tag)::value;
				// Mask keys outside the row's span or past the segment (only on
				// steps that cross an edge).
				if (kw0 < first_hi || kw0 + kWK - 1 > min(last_lo, seg_last))
				{
					const int hi_key = min(rlast, seg_last);
#pragma unroll
					for (int e = 0; e < 16; ++e)
					{
						const int k = kw0 + 8 * (e / 4) + 4 * h + (e % 4);
						if (k < rfirst || k > hi_key) sc[e] = -INFINITY;
					}
				}

				// Raise the row's offset when its scores outgrow it by more than
				// kLazy (or on its first visible key): rare, and O's rescale with it.
				float mx = sc[0];
#pragma unroll
				for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sc[e]);
				mx = max_with_other_half(mx);
				const bool grow = mx > kLazy || (m_off == -INFINITY && mx != -INFINITY);
				if (__builtin_amdgcn_ballot_w64(grow) != 0) // uniform
				{
					const bool fresh = m_off == -INFINITY;
					const float d = grow ? mx - kBias : 0.0f;
					const float alpha = fresh ? 0.0f : fast_exp2(-d); // 1 when the row does not grow
					if (grow) m_off = (fresh ? 0.0f : m_off) + d;
					const float ci = m_off == -INFINITY ? 0.0f : -m_off;
#pragma unroll
					for (int e = 0; e < 16; ++e) c_init[e] = ci;
#pragma unroll
					for (int b = 0; b < DBK; ++b) acc_o[b] *= alpha;
					l_acc *= alpha;
					sc -= d;
				}

				// P^T as the B operand, per 16-key half c (k-slot j holds key
				// 16 c + 8 (j / 4) + 4 h + j % 4, as in V^T above), and the row
				// sums. fp16: P rounded to fp16, the sums from the same rounded
				// weights. bf16: P split into bf16 hi + lo against the exact
				// bf16 V^T (no fp16 range limit on V), the sums in fp32.
#pragma unroll
				for (int c = 0; c < 2; ++c)
				{
					if constexpr (F16)
					{
						u32x4 pw;
#pragma unroll
						for (int q = 0; q < 4; ++q)
						{
							// (a scalar copy: clang's bit_cast of a vector element
							// reads element 0 whatever the index)
							const uint32_t w2 = pack_f16x2(fast_exp2(sc[8 * c + 2 * q]), fast_exp2(sc[8 * c + 2 * q + 1]));
							pw[q] = w2;
							l_acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w2), one2, l_acc, false);
						}
						const f16x8 pb = as_f16x8(pw);
						__builtin_amdgcn_s_setprio(1);
#pragma unroll
						for (int b = 0; b < DBK; ++b) acc_o[b] = mfma32x32x16(as_f16x8(vta[c][b]), pb, acc_o[b]);
						__builtin_amdgcn_s_setprio(0);
					}
					else
					{
						float w[8];
#pragma unroll
						for (int q = 0; q < 8; ++q)
						{
							w[q] = fast_exp2(sc[8 * c + q]);
							l_acc += w[q];
						}
						bf16x8 phi, plo;
						split_bf16x8(w, phi, plo);
						__builtin_amdgcn_s_setprio(1);
#pragma unroll
						for (int b = 0; b < DBK; ++b)
						{
							acc_o[b] = mfma32x32x16(as_bf16x8(vta[c][b]), phi, acc_o[b]);
							acc_o[b] = mfma32x32x16(as_bf16x8(vta[c][b]), plo, acc_o[b]);
						}
						__builtin_amdgcn_s_setprio(0);
					}
				}
			};

			// The key loop, in one of two instantiations: V in fp16 (the copy)
			// with P in fp16, or V in bf16 with P as bf16 hi + lo. With two row
			// groups the next step's K DMAs go out right after the step's
			// barrier and its V DMAs after the QK phase, so the address unit's
			// work is spread over the step (placements from all at the barrier
			// to all after the QK phase measured within 2 % of each other).
			auto key_loop = [&](auto f16_tag) __attribute__((always_inline))
			{
				for (int i = 0; i < n_steps; ++i)
				{
					int seg_last;
					const int kw0 = step_key(i, seg_last);
					dma_done(); // this step's tiles (this wavefront's DMAs) have landed
					if constexpr (RG > 1)
					{
						// Every wavefront's DMAs of this step have landed, and every
						// wavefront is done with the other stage (read in the last
						// step): the next step's loads go there.
						lds_reads_done();
						__syncthreads();
						if (i + 1 < n_steps) load_part(f16_tag, i + 1, 0, ND);
					}
					f32x16 sc;
					u32x4 vta[2][DBK]; // fp16 (the copy) or bf16 elements
					qk_phase(f16_tag, i, sc, vta);
					if (i + 1 < n_steps)
					{
						if constexpr (RG > 1)
							load_part(f16_tag, i + 1, ND, 2 * ND);
						else
						{
							// Both tiles are read: the next step's rows. A DMA's LDS
							// write is not ordered after earlier LDS reads still in
							// flight, so those complete first.
							lds_reads_done();
							load_tiles(f16_tag, i + 1);
						}
					}
					// The masking, the row maximum and the first half's weights
					// at a priority above the MFMA phases' 1 (the first P . V
					// block leaves it at 0): a wavefront there issues ahead of
					// the other wavefront of its SIMD issuing MFMAs (0.3-0.6 % less
					// time per prefill step).
					__builtin_amdgcn_s_setprio(2);
					soft_phase(f16_tag, kw0, seg_last, sc, vta);
					__builtin_amdgcn_s_setprio(0);
				}
			};
			if (use16)
				key_loop(std::true_type{});
			else
				key_loop(std::false_type{});

			// Merge the wavefronts: o = sum_w o_w 2^(m_w - M) / sum_w l_w 2^(m_w - M),
			// 0 when no key was seen (reference nn_ops.cpp:492). The row
			// statistics take the place of Q's hi half, the partial results that
			// of the tiles.
			float* s_m = reinterpret_cast<float*>(s_raw + S::kStats); // [kWaves][32]
			float* s_l = s_m + kWaves * 32;
			const float l_row = add_with_other_half(l_acc);
			// Every wavefront has left the key loop: the tiles are read (no DMA
			// is left: the last step issues none) and so is Q's hi half.
			__syncthreads();
			if (h == 0)
			{
				s_m[wave * 32 + r32] = m_off;
				s_l[wave * 32 + r32] = l_row;
			}
			__syncthreads();
			float* s_o = reinterpret_cast<float*>(s_raw);
			{
				// the key groups of this wavefront's row group: wavefronts rg kKG + w
				const float* sm = s_m + rg * kKG * 32 + r32;
				const float* sl = s_l + rg * kKG * 32 + r32;
				float M = sm[0];
#pragma unroll
				for (int w = 1; w < kKG; ++w) M = fmaxf(M, sm[w * 32]);
				float L = 0.0f, f_own = 0.0f;
#pragma unroll
				for (int w = 0; w < kKG; ++w)
				{
					const float mw = sm[w * 32];
					const float f = mw == -INFINITY ? 0.0f : fast_exp2(mw - M);
					L = fmaf(sl[w * 32], f, L);
					if (w == kg) f_own = f;
				}
				const float sc_own = L > 0.0f ? f_own / L : 0.0f;
				float* orow = s_o + (wave * 32 + r32) * OPITCH + 4 * h;
#pragma unroll
				for (int b = 0; b < DBK; ++b)
#pragma unroll
					for (int g = 0; g < 4; ++g)
						*reinterpret_cast<float4*>(orow + 32 * b + 8 * g) =
							make_float4(acc_o[b][4 * g] * sc_own, acc_o[b][4 * g + 1] * sc_own, acc_o[b][4 * g + 2] * sc_own,
							            acc_o[b][4 * g + 3] * sc_own);
			}
			__syncthreads();
			constexpr int Q4 = HD / 4; // float4s per row
			for (int idx = threadIdx.x; idx < kRows * Q4; idx += 64 * kWaves)
			{
				const int r = idx / Q4, d4 = idx % Q4;
				const int gr = row0 + r;
				if (gr >= n_rows) continue;
				// row r is row r % 32 of row group r / 32, kept by its kKG wavefronts
				const float* o0 = s_o + ((r / 32) * kKG * 32 + r % 32) * OPITCH + 4 * d4;
				float4 acc = *reinterpret_cast<const float4*>(o0);
#pragma unroll
				for (int w = 1; w < kKG; ++w)
				{
					const float4 v = *reinterpret_cast<const float4*>(o0 + w * 32 * OPITCH);
					acc.x += v.x;
					acc.y += v.y;
					acc.z += v.z;
					acc.w += v.w;
				}
				const size_t oi = static_cast<size_t>(gr / G) * q_stride + static_cast<size_t>(kvh * G + gr % G) * HD + 4 * d4;
				if (p.gate)
				{
					acc.x = gated(acc.x, p.gate, oi);
					acc.y = gated(acc.y, p.gate, oi + 1);
					acc.z = gated(acc.z, p.gate, oi + 2);
					acc.w = gated(acc.w, p.gate, oi + 3);
				}
				// non-temporal: written toward HBM as each work-group finishes,
				// not left dirty in L2 for the end of the kernel to write back
				store_stream(p.out + oi, acc);
			}
		}

		// head_dim 256 in 16-row tiles. 32 rows of 256 need 128 accumulator
		// registers per lane in 32 x 32 tiles, which leaves one wavefront per
		// SIMD; 16-row tiles on v_mfma_f32_16x16x32 need 64, so a work-group
		// of eight wavefronts — four key groups times two row groups of 16
		// rows — holds two per SIMD, Q (hi + lo) in registers, and the two
		// row groups share every K and V tile (loaded once per 32 rows, as
		// in the 32-row form; each row group issues half of every tile's
		// DMAs). LDS: one stage of tiles (128 KiB; two would not fit beside
		// Q's staging area), so a step waits for its tiles (barrier), takes
		// its scores and its V^T registers, waits until every wavefront has
		// (barrier), issues the next step's DMAs, and runs its softmax and
		// P.V from registers while they land.
		//   S^T = K . Q^T  per 16-key tile t: lane l holds keys key16(4 (l / 16)
		//                  + i) + 8 t of row l % 16 (two tiles, 8 scores);
		//   P^T            the lane's 8 weights are the B operand of a 32-key
		//                  product as they sit (k-slot 8 (l / 16) + j holds key
		//                  key16(4 (l / 16)) + j, j < 4, and that + 8 after), the
		//                  key order of block l / 16 of V's fp16 copy, whose
		//                  16 bytes per element are V^T's operand (one plain
		//                  LDS read); the bf16 V is read (ds_read_b64_tr_b16)
		//                  in that key order;
		//   O^T += V^T . P^T  16 tiles of 16 elements: lane l holds elements
		//                  16 dt + 4 (l / 16) + i of row l % 16.
		// The softmax, the lazy offset, V's fp16 copy and the final merge of
		// the key groups follow the 32-row kernel. (Measured against this
		// form on E's prefill, 25.8 ms: the tile halves pipelined — each
		// released and reloaded by its row group while the other half runs —
		// 53.6 ms with 23 registers spilled, whose reloads wait behind the
		// in-flight DMAs on the shared vector-memory count, and 28.0 ms
		// without spills, with each half's softmax and P.V on
		// v_mfma_f32_16x16x16; K released after the scores and V after P.V
		// in separate stages of one buffer 28.3 ms. A copy without the step
		// DMAs ran 16.9 ms.)
		constexpr int kH16 = 256;
		constexpr int kRows16 = 32, kWaves16 = 8;
		constexpr int kTile16 = kWK * kH16 * 2; // bytes of one K (or V) tile
		constexpr int kStage16 = kKG * 2 * kTile16; // 128 KiB
		constexpr int kQ16 = kRows16 * kH16 * 2; // one bf16 half of Q
		constexpr int kLds16 = kStage16 + 2 * kQ16; // 160 KiB
		constexpr int kOPitch16 = kH16 + 4;
		constexpr int kStats16 = kLds16 - 2 * kWaves16 * 16 * 4;
		static_assert(kWaves16 * 16 * kOPitch16 * 4 <= kStats16, "merge buffer layout");

		// 16-byte slot swizzle of V tile rows for the 16-row form: the
		// transposing reads of a 16-lane group cover 32 bytes of each of four
		// consecutive rows, and the four groups rows 4 apart; (row ^ row / 4)
		// % 4 puts all 16 rows' reads in distinct 64-byte bank groups.
		__device__ __forceinline__ int vswz16(int row) { return 4 * ((row ^ (row >> 2)) & 3); }

		// The score tiles' key order: tile t's row x (x < 16) is key key16(x) +
		// 8 t of the 32-key tile, i.e. tile 0 takes keys 0-7 and 16-23, tile 1
		// keys 8-15 and 24-31. Lane l then holds keys key16(4 (l / 16)) + i
		// (tile 0) and 8 more (tile 1), i < 4: the eight keys of block l / 16
		// of V's fp16 copy (f16_copy_index), which its P . V product takes as
		// they sit.
		__device__ __forceinline__ int key16(int x) { return x + 8 * (x >> 3); }
		// Tile rows swizzle as rows remap16(row) of a 16-row tile: the 16 rows
		// a score tile reads (and the V^T reads of a half-wavefront) fall on
		// 16 distinct ones.
		__device__ __forceinline__ int remap16(int row) { return (row & 7) | ((row >> 1) & 8); }

		template <int G>
		__global__ __launch_bounds__(64 * kWaves16) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill16_kernel(
			const prefill_params p)
		{
			constexpr int HD = kH16, KT = HD / 32, DT = HD / 16, LPK = HD / 8, KPL = 64 / LPK, NV = kWK / KPL,
			              ND = NV / 2;
			__shared__ __attribute__((aligned(16))) unsigned char s_raw[kLds16];

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
			const int kg = wave % kKG, rg = wave / kKG;
			const int r16 = lane & 15, g4 = lane >> 4;

			int bid = blockIdx.x;
			const int n_wg = gridDim.x;
			if ((n_wg & 7) == 0) bid = (bid & 7) * (n_wg >> 3) + (bid >> 3);
			const int kvh = bid / p.n_qtiles;
			const int j = bid % p.n_qtiles, half = (p.n_qtiles + 1) / 2;
			const int qt = j < half ? p.n_qtiles - 1 - j : j - half;

			const int n_rows = p.n_tok * G;
			const int row0 = qt * kRows16;
			const size_t q_stride = static_cast<size_t>(p.n_head) * HD;

			int kmin, kmax, first_hi, last_lo;
			{
				const int t0 = row0 / G, t1 = min(p.n_tok - 1, (row0 + kRows16 - 1) / G);
				attn_span(p.causal, p.window, p.pos0 + t0, p.n_seq, kmin, last_lo);
				attn_span(p.causal, p.window, p.pos0 + t1, p.n_seq, first_hi, kmax);
			}
			const int my_row = row0 + 16 * rg + r16;
			int rfirst = 1, rlast = 0;
			if (my_row < n_rows) attn_span(p.causal, p.window, p.pos0 + my_row / G, p.n_seq, rfirst, rlast);

			// V's fp16 copy, and the walk from kmin rounded down to 32, as in the
			// 32-row kernel.
			const bool use16 = p.V16 != nullptr && __builtin_amdgcn_readfirstlane(*p.n_bad) == 0 &&
			                   ((p.rows & 31) == 0 || kmax < p.rows);
			const int kbeg = use16 ? kmin & ~31 : kmin;
			const int span = kmax >= kmin ? kmax - kbeg + 1 : 0;
			const int rb0 = span > 0 ? kbeg % p.rows : 0;
			const int len1 = min(span, p.rows - rb0);
			const int len2 = span - len1;
			const int n1 = (len1 + kStep - 1) / kStep;
			const int n_steps = n1 + (len2 + kStep - 1) / kStep;
			const int wrap_key = kbeg + len1;

			const uint32_t row_bytes = static_cast<uint32_t>(p.kv_dim) * 2;
			const uint32_t head_bytes = static_cast<uint32_t>(kvh) * HD * 2;
			const char* kbase = static_cast<const char*>(p.K) + head_bytes;
			const char* vbase = use16 ? static_cast<const char*>(p.V16) + 8 * head_bytes
			                          : static_cast<const char*>(p.V) + head_bytes;

			auto step_key = [&](int i, int& seg_last) __attribute__((always_inline)) -> int
			{
				const bool second = i >= n1;
				seg_last = second ? kmax : wrap_key - 1;
				return (second ? wrap_key + (i - n1) * kStep : kbeg + i * kStep) + kg * kWK;
			};
			const uint32_t step_bytes = static_cast<uint32_t>(kStep) * row_bytes;
			const uint32_t seg1_off = static_cast<uint32_t>(rb0 + kg * kWK) * row_bytes;
			const uint32_t seg2_off = static_cast<uint32_t>(kg * kWK) * row_bytes - static_cast<uint32_t>(n1) * step_bytes;
			const uint32_t seg1_end = static_cast<uint32_t>(rb0 + len1 - 1) * row_bytes + HD * 2;
			const uint32_t seg2_end = static_cast<uint32_t>(kmax - wrap_key) * row_bytes + HD * 2;
			auto group_end = [&](int last_row) __attribute__((always_inline)) -> uint32_t
			{
				return static_cast<uint32_t>(last_row >> 5) * 32 * row_bytes + 24 * row_bytes + 16 * HD;
			};
			const uint32_t v_seg1_end = use16 ? group_end(rb0 + len1 - 1) : seg1_end;
			const uint32_t v_seg2_end = use16 ? group_end(kmax - wrap_key) : seg2_end;
			auto step_rsrc = [&](int i, const char* base, bool is_v) __attribute__((always_inline))
			{
				const bool second = i >= n1;
				const uint32_t off = (second ? seg2_off : seg1_off) + static_cast<uint32_t>(i) * step_bytes;
				const uint32_t end = is_v ? (second ? v_seg2_end : v_seg1_end) : (second ? seg2_end : seg1_end);
				const uint32_t n = __builtin_amdgcn_readfirstlane(end > off ? end - off : 0u);
				return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base + off), 0, static_cast<int>(n),
				                                         kBufferFlags);
			};

			// The key group's K tile, then its V tile; the two row groups split
			// each tile's DMAs (row group rg: rows 16 rg .. 16 rg + 15).
			// (tile rows swizzle as rows remap16(row): see the score tiles' key
			// order below)
			const int t_row = lane / LPK;
			uint16_t* const kt = reinterpret_cast<uint16_t*>(s_raw) + kg * 2 * kWK * HD;
			uint16_t* const vt = kt + kWK * HD;
			auto load_tiles = [&](auto f16_tag, int i) __attribute__((always_inline))
			{
				constexpr bool F16 = decltype(f16_tag)::value;
				const __amdgpu_buffer_rsrc_t rk = step_rsrc(i, kbase, false);
				const __amdgpu_buffer_rsrc_t rv = step_rsrc(i, vbase, true);
#pragma unroll
				for (int e = 0; e < 2 * ND; ++e)
				{
					const bool is_v = e >= ND;
					const int jj = rg * ND + (is_v ? e - ND : e);
					const int row = jj * KPL + t_row;
					const uint32_t rb = static_cast<uint32_t>(row) * row_bytes;
					if (is_v && F16) // tile byte 1024 jj + 16 l: block jj / 4, 16 kv_dim bytes per block
						load_lds16_grouped(rv, vt, jj, (jj >> 2) * 8 * row_bytes + 1024u * (jj & 3) + 16u * lane);
					else if (is_v)
						load_lds16_grouped(rv, vt, jj,
						                   rb + 16u * static_cast<uint32_t>((lane % LPK) ^ vswz16(remap16(row))));
					else
						load_lds16_grouped(rk, kt, jj,
						                   rb + 16u * static_cast<uint32_t>((lane % LPK) ^ kswz<HD>(remap16(row))));
				}
			};
			static_assert(16 * HD == 4096, "the fp16 copy's DMA offsets assume 4 KiB blocks");
			if (n_steps > 0)
			{
				if (use16)
					load_tiles(std::true_type{}, 0);
				else
					load_tiles(std::false_type{}, 0);
			}

			// Q, pre-scaled into log2 units, as bf16 hi + lo in LDS (the K
			// tiles' layout).
			uint16_t* s_qhi = reinterpret_cast<uint16_t*>(s_raw + kStage16);
			uint16_t* s_qlo = reinterpret_cast<uint16_t*>(s_raw + kStage16 + kQ16);
			stage_q<HD, G, kRows16, 64 * kWaves16>(p.q, q_stride, p.qscale, kvh, row0, n_rows, s_qhi, s_qlo);
			__syncthreads();
			// Q^T as the B operand of k-step kk: lane l holds row l % 16 of the
			// row group, elements 32 kk + 8 (l / 16) .. + 8.
			bf16x8 qhi[KT], qlo[KT];
			{
				const int qrow = 16 * rg + r16;
#pragma unroll
				for (int kk = 0; kk < KT; ++kk)
				{
					const int off = qrow * HD + 8 * ((4 * kk + g4) ^ kswz<HD>(qrow));
					qhi[kk] = *reinterpret_cast<const bf16x8*>(s_qhi + off);
					qlo[kk] = *reinterpret_cast<const bf16x8*>(s_qlo + off);
				}
			}

			f32x4 acc_o[DT];
#pragma unroll
			for (int d = 0; d < DT; ++d) acc_o[d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
			float l_acc = 0.0f, m_off = -INFINITY, c_init = 0.0f;
			const f16x2 one2 = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};

			// V^T for O^T tile dt (bf16 V): keys key16(4 (l / 16)) + r_off .. + 3
			// of element 16 dt + l % 16 (r_off = 0: k-slots 8 (l / 16) .. + 3 of
			// the product; r_off = 8: the next four).
			auto vt_half = [&](int dt, int r_off) __attribute__((always_inline)) -> u32x2
			{
				const int col = 16 * dt + 4 * (r16 & 3);
				const int slot = col >> 3, in = col & 7;
				// (remap16(ra) is 4 (l / 16) + (l % 16) / 4 for both r_off)
				const int ra = key16(4 * g4) + r_off + (r16 >> 2);
				return tr_read(vt + ra * HD + 8 * (slot ^ vswz16(4 * g4 + (r16 >> 2))) + in);
			};

			auto key_loop = [&](auto f16_tag) __attribute__((always_inline))
			{
				constexpr bool F16 = decltype(f16_tag)::value;
				for (int i = 0; i < n_steps; ++i)
				{
					int seg_last;
					const int kw0 = step_key(i, seg_last);
					dma_done();
					__syncthreads(); // every DMA of this step has landed

					f32x4 sc[2];
					u32x4 vta[DT];
					__builtin_amdgcn_s_setprio(1);
#pragma unroll
					for (int t = 0; t < 2; ++t)
					{
						sc[t] = f32x4{c_init, c_init, c_init, c_init};
						// (remap16(krow) is r16 in both tiles, so the row's swizzle
						// is kswz(r16))
						const int krow = key16(r16) + 8 * t;
#pragma unroll
						for (int kk = 0; kk < KT; ++kk)
						{
							const bf16x8 a =
								*reinterpret_cast<const bf16x8*>(kt + krow * HD + 8 * ((4 * kk + g4) ^ kswz<HD>(r16)));
							sc[t] = mfma16x16x32(a, qhi[kk], sc[t]);
							sc[t] = mfma16x16x32(a, qlo[kk], sc[t]);
						}
					}
#pragma unroll
					for (int d = 0; d < DT; ++d)
					{
						if constexpr (F16) // block l / 16 of the copy's tile: one plain read
							vta[d] = *reinterpret_cast<const u32x4*>(vt + (g4 * HD + 16 * d + r16) * 8);
						else
						{
							const u32x2 lo = vt_half(d, 0), hi = vt_half(d, 8);
							vta[d] = u32x4{lo.x, lo.y, hi.x, hi.y};
						}
					}
					__builtin_amdgcn_s_setprio(0);
					lds_reads_done();
					__syncthreads(); // every wavefront is done with this stage
					if (i + 1 < n_steps) load_tiles(f16_tag, i + 1);

					// Mask keys outside the row's span or past the segment (only
					// on steps that cross an edge).
					if (kw0 < first_hi || kw0 + kWK - 1 > min(last_lo, seg_last))
					{
						const int hi_key = min(rlast, seg_last);
#pragma unroll
						for (int t = 0; t < 2; ++t)
#pragma unroll
							for (int e = 0; e < 4; ++e)
							{
								const int k = kw0 + key16(4 * g4 + e) + 8 * t;
								if (k < rfirst || k > hi_key) sc[t][e] = -INFINITY;
							}
					}
					float mx = fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
					                 fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
					{
						const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false,
						                                                false);
						mx = max_with_other_half(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
					}
					const bool grow = mx > kLazy || (m_off == -INFINITY && mx != -INFINITY);
					if (__builtin_amdgcn_ballot_w64(grow) != 0)
					{
						const bool fresh = m_off == -INFINITY;
						const float d = grow ? mx - kBias : 0.0f;
						const float alpha = fresh ? 0.0f : fast_exp2(-d);
						if (grow) m_off = (fresh ? 0.0f : m_off) + d;
						c_init = m_off == -INFINITY ? 0.0f : -m_off;
#pragma unroll
						for (int dd = 0; dd < DT; ++dd) acc_o[dd] *= alpha;
						l_acc *= alpha;
						sc[0] -= d;
						sc[1] -= d;
					}

					if constexpr (F16)
					{
						u32x4 pw;
#pragma unroll
						for (int q = 0; q < 4; ++q)
						{
							const int t = q >> 1, e = 2 * (q & 1);
							const uint32_t w2 = pack_f16x2(fast_exp2(sc[t][e]), fast_exp2(sc[t][e + 1]));
							pw[q] = w2;
							l_acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w2), one2, l_acc, false);
						}
						const f16x8 pb = as_f16x8(pw);
						__builtin_amdgcn_s_setprio(1);
#pragma unroll
						for (int d = 0; d < DT; ++d) acc_o[d] = mfma16x16x32(as_f16x8(vta[d]), pb, acc_o[d]);
						__builtin_amdgcn_s_setprio(0);
					}
					else
					{
						float w[8];
#pragma unroll
						for (int q = 0; q < 8; ++q)
						{
							w[q] = fast_exp2(sc[q >> 2][q & 3]);
							l_acc += w[q];
						}
						bf16x8 phi, plo;
						split_bf16x8(w, phi, plo);
						__builtin_amdgcn_s_setprio(1);
#pragma unroll
						for (int d = 0; d < DT; ++d)
						{
							acc_o[d] = mfma16x16x32(as_bf16x8(vta[d]), phi, acc_o[d]);
							acc_o[d] = mfma16x16x32(as_bf16x8(vta[d]), plo, acc_o[d]);
						}
						__builtin_amdgcn_s_setprio(0);
					}
				}
			};
			if (use16)
				key_loop(std::true_type{});
			else
				key_loop(std::false_type{});

			// Merge the key groups of each row group (as the 32-row kernel).
			float* s_m = reinterpret_cast<float*>(s_raw + kStats16); // [kWaves16][16]
			float* s_l = s_m + kWaves16 * 16;
			const float l_row = add_with_other_half(add_with_other_row(l_acc));
			__syncthreads(); // the tiles and Q's staging area are free
			if (g4 == 0)
			{
				s_m[wave * 16 + r16] = m_off;
				s_l[wave * 16 + r16] = l_row;
			}
			__syncthreads();
			float* s_o = reinterpret_cast<float*>(s_raw);
			{
				const float* sm = s_m + rg * kKG * 16 + r16;
				const float* sl = s_l + rg * kKG * 16 + r16;
				float M = sm[0];
#pragma unroll
				for (int w = 1; w < kKG; ++w) M = fmaxf(M, sm[w * 16]);
				float L = 0.0f, f_own = 0.0f;
#pragma unroll
				for (int w = 0; w < kKG; ++w)
				{
					const float mw = sm[w * 16];
					const float f = mw == -INFINITY ? 0.0f : fast_exp2(mw - M);
					L = fmaf(sl[w * 16], f, L);
					if (w == kg) f_own = f;
				}
				const float sc_own = L > 0.0f ? f_own / L : 0.0f;
				float* orow = s_o + (wave * 16 + r16) * kOPitch16 + 4 * g4;
#pragma unroll
				for (int d = 0; d < DT; ++d)
					*reinterpret_cast<float4*>(orow + 16 * d) =
						make_float4(acc_o[d][0] * sc_own, acc_o[d][1] * sc_own, acc_o[d][2] * sc_own, acc_o[d][3] * sc_own);
			}
			__syncthreads();
			constexpr int Q4 = HD / 4;
			for (int idx = threadIdx.x; idx < kRows16 * Q4; idx += 64 * kWaves16)
			{
				const int r = idx / Q4, d4 = idx % Q4;
				const int gr = row0 + r;
				if (gr >= n_rows) continue;
				// row r is row r % 16 of row group r / 16, kept by its kKG wavefronts
				const float* o0 = s_o + ((r / 16) * kKG * 16 + r % 16) * kOPitch16 + 4 * d4;
				float4 acc = *reinterpret_cast<const float4*>(o0);
#pragma unroll
				for (int w = 1; w < kKG; ++w)
				{
					const float4 v = *reinterpret_cast<const float4*>(o0 + w * 16 * kOPitch16);
					acc.x += v.x;
					acc.y += v.y;
					acc.z += v.z;
					acc.w += v.w;
				}
				const size_t oi = static_cast<size_t>(gr / G) * q_stride + static_cast<size_t>(kvh * G + gr % G) * HD + 4 * d4;
				if (p.gate)
				{
					acc.x = gated(acc.x, p.gate, oi);
					acc.y = gated(acc.y, p.gate, oi + 1);
					acc.z = gated(acc.z, p.gate, oi + 2);
					acc.w = gated(acc.w, p.gate, oi + 3);
				}
				// non-temporal: written toward HBM as each work-group finishes,
				// not left dirty in L2 for the end of the kernel to write back
				store_stream(p.out + oi, acc);
			}
		}

		bool launch_hd256_16(prefill_params p, int group, hipStream_t stream)
		{
			p.n_qtiles = (p.n_tok * group + kRows16 - 1) / kRows16;
			const dim3 grid(p.n_qtiles * p.n_kv), block(64 * kWaves16);
			switch (group)
			{
			case 1: prefill16_kernel<1><<<grid, block, 0, stream>>>(p); return true;
			case 2: prefill16_kernel<2><<<grid, block, 0, stream>>>(p); return true;
			case 4: prefill16_kernel<4><<<grid, block, 0, stream>>>(p); return true;
			case 8: prefill16_kernel<8><<<grid, block, 0, stream>>>(p); return true;
			default: return false;
			}
		}

		template <int HD, int RG>
		bool launch_hd(prefill_params p, int group, hipStream_t stream)
		{
			using S = prefill_shape<HD, RG>;
			p.n_qtiles = (p.n_tok * group + S::ROWS - 1) / S::ROWS;
			const dim3 grid(p.n_qtiles * p.n_kv), block(64 * S::WAVES);
			switch (group)
			{
			case 1: prefill_kernel<HD, 1, RG><<<grid, block, 0, stream>>>(p); return true;
			case 2: prefill_kernel<HD, 2, RG><<<grid, block, 0, stream>>>(p); return true;
			case 4: prefill_kernel<HD, 4, RG><<<grid, block, 0, stream>>>(p); return true;
			case 8: prefill_kernel<HD, 8, RG><<<grid, block, 0, stream>>>(p); return true;
			default: return false;
			}
		}
	}

	bool launch_prefill(prefill_params p, int head_dim, int group, bool bf16, hipStream_t stream)
	{
		if (!bf16) return false;
		switch (head_dim)
		{
		case 64: return launch_hd<64, 2>(p, group, stream);
		case 128: return launch_hd<128, 2>(p, group, stream);
		case 256: return launch_hd256_16(p, group, stream);
		default: return false;
		}
	}
}
