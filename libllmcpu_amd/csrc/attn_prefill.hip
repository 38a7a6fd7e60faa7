// Flash attention on CDNA4 MFMA for a batch of query tokens (nnc's batch
// path, reference src/libnnc/model.cpp:1750-1757, and the chunked prefill of
// a long prompt), BF16 K/V.
//
// Rows of the problem are (token, query head) pairs of one KV head, token
// major, so the heads of a GQA group sit in adjacent rows and share every key
// the work-group reads. Grid: n_kv * n_qtiles work-groups of 4 wavefronts; a
// work-group owns ROWS = 16 * NB rows and walks its key range in steps of
// 128 keys, wavefront w taking keys 32w .. 32w + 31 of each step for all of
// the work-group's rows. Each wavefront therefore reads a disjoint quarter of
// the keys straight from L2 into registers (no K/V tile is copied to every
// wavefront), keeps its own online softmax, and the four partial results
// merge once, in LDS, at the end:
//   S^T = K . Q^T      v_mfma_f32_16x16x32_bf16 with K's rows as the A
//                      operand exactly as loaded (16 contiguous bytes per
//                      lane) and Q^T as B, split into bf16 hi + lo so the
//                      product against the exact bf16 K is near-fp32. The
//                      accumulator starts at -m (the row's running offset),
//                      so the scores come out already shifted;
//   softmax            in fp32 and log2 units (Q is pre-scaled by
//                      scale * log2 e). The offset m is raised only when a
//                      row's scores exceed it by more than 8, so weights stay
//                      in (0, 256] and the O rescale is rare;
//   O^T += V^T . P^T   v_mfma_f32_16x16x32_f16. The wavefront's 32 V rows go
//                      to its own LDS tile as fp16 (bf16 -> fp16 is exact up
//                      to 65504; larger magnitudes saturate there) and come
//                      back transposed with ds_read_b64_tr_b16; P (fp16,
//                      rounded to nearest) is the B operand straight from the
//                      score registers (key order permuted to match). The
//                      row sums l come from the same rounded P through one
//                      more MFMA against a block of ones, so numerator and
//                      denominator see identical weights.
// The next step's K and V loads are in flight during the current step's
// math. Masking is applied only to steps that cross some row's span edge;
// keys are never read out of bounds (rows are clamped into the valid range
// and masked keys weigh exactly 0). The final merge sums the wavefronts in a
// fixed order, so results are the same run to run.
#include "device_common.h"
#include "kernels.h"

namespace nnchip
{
	namespace
	{
		constexpr int kWaves = 4; // wavefronts per work-group
		constexpr int kWK = 32; // keys per wavefront per step
		constexpr int kStep = kWaves * kWK; // keys per work-group step
		constexpr float kLazy = 8.0f; // max growth of a row's scores over its offset, log2 units
		constexpr int kBufferFlags = 0x00020000; // buffer descriptor word 3: raw 32-bit data

		// Wavefronts per SIMD: two let one wavefront's softmax and loads overlap
		// the other's MFMAs, and cap a wavefront at 256 registers.
		constexpr int kWpe = 2;

		// Per head_dim, within a wavefront's 256 registers: 16-row blocks per
		// work-group (NB), whether Q's hi half also waits in LDS (the lo half
		// always does), and whether K streams into LDS a step ahead (else into
		// registers at the start of its step).
		template <int HD>
		struct prefill_cfg;
		template <>
		struct prefill_cfg<64>
		{
			static constexpr int NB = 2, WPE = 2;
			static constexpr bool QHI_LDS = false, K_LDS = true;
		};
		template <>
		struct prefill_cfg<128>
		{
			static constexpr int NB = 2, WPE = 2;
			static constexpr bool QHI_LDS = false, K_LDS = true;
		};
		template <>
		struct prefill_cfg<256>
		{
			static constexpr int NB = 1, WPE = 2;
			static constexpr bool QHI_LDS = false, K_LDS = false; // LDS-bound: two work-groups per CU must fit
		};

		template <int HD, int NB, bool QHI_LDS, bool K_LDS>
		struct prefill_shape
		{
			static constexpr int KK = HD / 32; // k-steps of the QK MFMA
			static constexpr int DB = HD / 16; // 16-row d blocks of O^T
			static constexpr int ROWS = 16 * NB; // rows per work-group
			static constexpr int LPK = HD / 8; // lanes per V row (16 bytes each)
			static constexpr int KPL = 64 / LPK; // V rows per load
			static constexpr int NV = kWK / KPL; // V loads per step
			static constexpr int OPITCH = HD + 4; // floats per row in the final merge
			static constexpr int QPITCH = HD + 8; // bf16 per row of Q's halves in LDS
			static constexpr int kVBytes = kWaves * kWK * HD * 2; // per-wavefront V tiles, bf16
			static constexpr int kQBytes = (QHI_LDS ? 2 : 1) * ROWS * QPITCH * 2; // lo rows, then hi rows
			static constexpr int kOBytes = kWaves * ROWS * OPITCH * 4;
			static constexpr int kKBytes = K_LDS ? kWaves * kWK * HD * 2 : 0; // per-wavefront K tiles, bf16
			static constexpr int kLoop = kVBytes + kKBytes + kQBytes;
			static constexpr int kLds = kLoop > kOBytes ? kLoop : kOBytes;
			static_assert(NV >= 1 && KPL * NV == kWK, "unsupported prefill shape");
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

		// 16-byte slot swizzle of row `row` of a V tile (an even XOR, so a
		// 32-byte pair stays together): the transposing reads of four (and
		// eight) consecutive rows at one element offset land in distinct banks.
		template <int HD>
		__device__ __forceinline__ int vswz(int row)
		{
			return HD == 64 ? 2 * ((row >> 1) & 3) : 2 * (row & 7);
		}

		// 16 bytes per lane from a buffer straight into LDS: lane l's bytes land
		// at lds + 16 l (the LDS address is uniform over the wavefront).
		__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t rsrc, void* lds, uint32_t voffset)
		{
			typedef __attribute__((address_space(3))) void* lds_ptr;
			__builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr)lds, 16, voffset, 0, 0, 0);
		}

		// 16-byte slot swizzle of row `row` of a K tile: the A-operand reads of
		// 16 consecutive rows at one slot land in distinct banks.
		template <int HD>
		__device__ __forceinline__ int kswz(int row)
		{
			return HD == 64 ? (row >> 1) & 7 : row & 15;
		}

		// Eight bf16 (one 16-byte load) -> eight fp16, exact up to 65504.
		__device__ __forceinline__ u32x4 bf16x8_to_f16x8(const u32x4& b)
		{
			return u32x4{pack_f16x2_rtz(bf16_lo(b.x), bf16_hi(b.x)), pack_f16x2_rtz(bf16_lo(b.y), bf16_hi(b.y)),
			             pack_f16x2_rtz(bf16_lo(b.z), bf16_hi(b.z)), pack_f16x2_rtz(bf16_lo(b.w), bf16_hi(b.w))};
		}

		// acc *= s for an accumulator held in AGPRs: each element goes through
		// a temporary VGPR inside the asm, so the compiler keeps the O
		// accumulators in AGPRs instead of copying them to VGPRs around the
		// (rare) rescale.
		__device__ __forceinline__ void scale_in_agpr(f32x4& acc, float s)
		{
#pragma unroll
			for (int e = 0; e < 4; ++e)
			{
				float x = acc[e], t;
				asm volatile("v_accvgpr_read_b32 %1, %0\n\tv_mul_f32 %1, %1, %2\n\tv_accvgpr_write_b32 %0, %1"
				             : "+a"(x), "=&v"(t)
				             : "v"(s));
				acc[e] = x;
			}
		}

		template <int HD, int G>
		__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kWpe, kWpe))) void prefill_kernel(
			const prefill_params p)
		{
			static_assert(prefill_cfg<HD>::WPE == kWpe, "one occupancy for every head_dim");
			constexpr int NB = prefill_cfg<HD>::NB;
			constexpr bool QHI_LDS = prefill_cfg<HD>::QHI_LDS, K_LDS = prefill_cfg<HD>::K_LDS;
			using S = prefill_shape<HD, NB, QHI_LDS, K_LDS>;
			constexpr int KK = S::KK, DB = S::DB, ROWS = S::ROWS, LPK = S::LPK, KPL = S::KPL, NV = S::NV,
			              OPITCH = S::OPITCH, QPITCH = S::QPITCH;

			// V tiles and Q's lo half during the key loop, then the merge buffer.
			__shared__ __attribute__((aligned(16))) unsigned char s_raw[S::kLds];
			__shared__ float s_m[kWaves][ROWS];
			__shared__ float s_l[kWaves][ROWS];

			const int lane = threadIdx.x & 63;
			const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); // uniform: keeps step control scalar
			const int col = lane & 15;
			const int grp = lane >> 4;

			// Work-groups of one KV head run on one XCD (blockIdx.x % 8 picks
			// the XCD), so its K/V rows are shared through that XCD's L2; within
			// a head, the query tiles with the most keys start first.
			int bid = blockIdx.x;
			const int n_wg = gridDim.x;
			if ((n_wg & 7) == 0) bid = (bid & 7) * (n_wg >> 3) + (bid >> 3);
			const int kvh = bid / p.n_qtiles;
			const int qt = p.n_qtiles - 1 - bid % p.n_qtiles;

			const int n_rows = p.n_tok * G;
			const int row0 = qt * ROWS;
			const size_t q_stride = static_cast<size_t>(p.n_head) * HD;

			// The work-group's key range [kmin, kmax], and [first_hi, last_lo],
			// the keys every one of its rows sees (span ends grow with the
			// position).
			int kmin, kmax, first_hi, last_lo;
			{
				const int t0 = row0 / G, t1 = min(p.n_tok - 1, (row0 + ROWS - 1) / G);
				attn_span(p.causal, p.window, p.pos0 + t0, p.n_seq, kmin, last_lo);
				attn_span(p.causal, p.window, p.pos0 + t1, p.n_seq, first_hi, kmax);
			}
			// Each lane's rows (one per 16-row block): their spans.
			int rfirst[NB], rlast[NB];
#pragma unroll
			for (int nb = 0; nb < NB; ++nb)
			{
				const int r = row0 + 16 * nb + col;
				if (r < n_rows)
					attn_span(p.causal, p.window, p.pos0 + r / G, p.n_seq, rfirst[nb], rlast[nb]);
				else
				{
					rfirst[nb] = 1;
					rlast[nb] = 0; // no key
				}
			}

			// Q^T as the B operand, pre-scaled into log2 units, bf16 hi + lo. The
			// lo half (and, where registers are short, the hi half) waits in LDS
			// at the address the same lane reads it back from.
			bf16x8 qhi[QHI_LDS ? 1 : NB][KK];
			uint16_t* s_q = reinterpret_cast<uint16_t*>(s_raw + S::kVBytes + S::kKBytes);
			auto q_lds = [&](int half, int nb, int kk) __attribute__((always_inline)) -> bf16x8*
			{
				return reinterpret_cast<bf16x8*>(s_q + (half * ROWS + 16 * nb + col) * QPITCH + 32 * kk + 8 * grp);
			};
#pragma unroll
			for (int nb = 0; nb < NB; ++nb)
			{
				const int r = row0 + 16 * nb + col;
				const bool ok = r < n_rows;
				const float* qp =
					p.q + (ok ? static_cast<size_t>(r / G) * q_stride + static_cast<size_t>(kvh * G + r % G) * HD : 0);
#pragma unroll
				for (int kk = 0; kk < KK; ++kk)
				{
					float x[8];
					if (ok)
					{
						const float4 a = *reinterpret_cast<const float4*>(qp + 32 * kk + 8 * grp);
						const float4 b = *reinterpret_cast<const float4*>(qp + 32 * kk + 8 * grp + 4);
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
					*q_lds(0, nb, kk) = lo;
					if constexpr (QHI_LDS)
						*q_lds(1, nb, kk) = hi;
					else
						qhi[QHI_LDS ? 0 : nb][kk] = hi;
				}
			}

			f32x4 acc_o[DB][NB];
			f32x4 acc_l[NB];
			float m_off[NB]; // each row's score offset (-inf until it has seen a key)
			f32x4 c_init[NB]; // S^T's accumulator start: -m_off, or 0 before the first key
#pragma unroll
			for (int nb = 0; nb < NB; ++nb)
			{
#pragma unroll
				for (int db = 0; db < DB; ++db) acc_o[db][nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
				acc_l[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
				m_off[nb] = -INFINITY;
				c_init[nb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
			}

			// K and V are read through buffer descriptors, whose range check
			// returns zeros for an offset past the descriptor's end without
			// touching memory. The work-group's keys kmin .. kmax sit in rows
			// rb0 .. rb0 + (kmax - kmin) of a full buffer, or wrap a ring once.
			// A step reads from a descriptor based at its first row whose range
			// ends at kmax's row (or the ring's end), so keys past kmax read as
			// 0 (their weight is 0 as well); a step past the ring's end reads
			// the wrapped rows the same way. The one step that may straddle the
			// end computes each lane's row instead. Byte offsets are 32-bit (the
			// host keeps a buffer under 2 GiB); the per-lane parts are
			// loop-invariant.
			const uint32_t row_bytes = static_cast<uint32_t>(p.kv_dim) * 2;
			const uint32_t head_bytes = static_cast<uint32_t>(kvh) * HD * 2;
			const int rb0 = kmax >= kmin ? kmin % p.rows : 0;
			const int last_row = rb0 + (kmax - kmin); // kmax's row before wrapping
			const bool wraps = last_row >= p.rows;
			// Bytes from row 0 of this head to the end of the main / wrapped range.
			const int64_t end_main = static_cast<int64_t>(wraps ? p.rows : last_row + 1) * row_bytes - head_bytes;
			const int64_t end_wrap = wraps ? static_cast<int64_t>(last_row - p.rows + 1) * row_bytes - head_bytes : 0;
			const int64_t end_ring = static_cast<int64_t>(p.rows) * row_bytes - head_bytes;
			const char* kbase = static_cast<const char*>(p.K) + head_bytes;
			const char* vbase = static_cast<const char*>(p.V) + head_bytes;
			auto rsrc = [&](const char* base, int64_t row, int64_t end) __attribute__((always_inline))
			{
				const int64_t off = row * row_bytes;
				const int64_t n = end - off;
				return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base + off), 0,
				                                         static_cast<int>(n > 0 ? n : 0), kBufferFlags);
			};
			// Step i's wavefront block starts at unwrapped row r: its descriptor,
			// or, when the block straddles the ring's end, none.
			auto step_rsrc = [&](int i, const char* base, int& r) __attribute__((always_inline))
			{
				r = rb0 + i * kStep + wave * kWK;
				return r >= p.rows ? rsrc(base, r - p.rows, end_wrap) : rsrc(base, r, end_main);
			};
			auto straddles = [&](int r) __attribute__((always_inline)) { return r < p.rows && r + kWK > p.rows; };
			// A straddling block's lane offset for block row o, relative to row 0
			// of the ring (out of range past kmax).
			auto ring_off = [&](int r, int o, uint32_t col_bytes) __attribute__((always_inline)) -> uint32_t
			{
				int row = r + o;
				const bool ok = row <= last_row;
				if (row >= p.rows) row -= p.rows;
				return ok ? static_cast<uint32_t>(row) * row_bytes + col_bytes : 0x80000000u;
			};

			const int v_row = lane / LPK; // a lane's tile row within one 16-byte-per-lane load

			// K as the A operand: lane (grp, col) takes key col of a 16-key block,
			// elements 32 kk + 8 grp .. + 8 (16-byte slot 4 kk + grp of the row).
			// K_LDS: the wavefront's 32 rows stream into its LDS tile like V's
			// (slot s of row r at s ^ kswz(r)), a step ahead of their use;
			// otherwise they load into registers at the start of the step.
			uint16_t* kt = reinterpret_cast<uint16_t*>(s_raw + S::kVBytes) + wave * kWK * HD;
			uint32_t k_off[2];
#pragma unroll
			for (int mb = 0; mb < 2; ++mb) k_off[mb] = static_cast<uint32_t>(16 * mb + col) * row_bytes + 16u * grp;
			uint32_t k_col[NV];
#pragma unroll
			for (int j = 0; j < NV; ++j) k_col[j] = 16u * static_cast<uint32_t>((lane % LPK) ^ kswz<HD>(j * KPL + v_row));
			u32x4 kreg[K_LDS ? 1 : 2][KK];
			auto load_k_lds = [&](int i) __attribute__((always_inline))
			{
				int r;
				const __amdgpu_buffer_rsrc_t rk = step_rsrc(i, kbase, r);
				if (!straddles(r))
				{
#pragma unroll
					for (int j = 0; j < NV; ++j)
						load_lds16(rk, kt + j * KPL * HD, static_cast<uint32_t>(j * KPL + v_row) * row_bytes + k_col[j]);
				}
				else
				{
					const __amdgpu_buffer_rsrc_t ring = rsrc(kbase, 0, end_ring);
#pragma unroll
					for (int j = 0; j < NV; ++j)
						load_lds16(ring, kt + j * KPL * HD, ring_off(r, j * KPL + v_row, k_col[j]));
				}
			};
			auto load_k = [&](int i) __attribute__((always_inline))
			{
				if constexpr (K_LDS)
				{
					load_k_lds(i);
					return;
				}
				int r;
				const __amdgpu_buffer_rsrc_t rk = step_rsrc(i, kbase, r);
				if (!straddles(r))
				{
#pragma unroll
					for (int mb = 0; mb < 2; ++mb)
#pragma unroll
						for (int kk = 0; kk < KK; ++kk)
							kreg[K_LDS ? 0 : mb][kk] =
								__builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, k_off[mb] + 64u * kk, 0, 0));
				}
				else
				{
					const __amdgpu_buffer_rsrc_t ring = rsrc(kbase, 0, end_ring);
#pragma unroll
					for (int mb = 0; mb < 2; ++mb)
					{
						const uint32_t off = ring_off(r, 16 * mb + col, 16u * grp);
#pragma unroll
						for (int kk = 0; kk < KK; ++kk)
							kreg[K_LDS ? 0 : mb][kk] =
								__builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ring, off + 64u * kk, 0, 0));
					}
				}
			};

			// V straight into the wavefront's LDS tile (rows of HD bf16, no
			// padding): load j fills tile rows j KPL .. + KPL, lane l the 16
			// bytes at l * 16, i.e. row j KPL + l / LPK, 16-byte slot l % LPK,
			// which holds the row's segment (l % LPK) ^ vswz(row). The swizzle
			// keeps the transposing reads of 4 (8) rows in distinct banks.
			uint16_t* vt = reinterpret_cast<uint16_t*>(s_raw) + wave * kWK * HD;
			uint32_t v_col[NV];
#pragma unroll
			for (int j = 0; j < NV; ++j) v_col[j] = 16u * static_cast<uint32_t>((lane % LPK) ^ vswz<HD>(j * KPL + v_row));
			auto load_v = [&](int i) __attribute__((always_inline))
			{
				int r;
				const __amdgpu_buffer_rsrc_t rv = step_rsrc(i, vbase, r);
				if (!straddles(r))
				{
#pragma unroll
					for (int j = 0; j < NV; ++j)
						load_lds16(rv, vt + j * KPL * HD, static_cast<uint32_t>(j * KPL + v_row) * row_bytes + v_col[j]);
				}
				else
				{
					const __amdgpu_buffer_rsrc_t ring = rsrc(vbase, 0, end_ring);
#pragma unroll
					for (int j = 0; j < NV; ++j)
						load_lds16(ring, vt + j * KPL * HD, ring_off(r, j * KPL + v_row, v_col[j]));
				}
			};
			const int n_steps = kmax >= kmin ? (kmax - kmin) / kStep + 1 : 0;

			// fp16 1.0 in every element: the A operand that sums P over keys.
			const f16x8 ones = as_f16x8(u32x4{0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u});

			// scores: S^T - m_off for both 16-key blocks, then the next K loads.
			auto scores = [&](int i, f32x4 (&sc)[2][NB]) __attribute__((always_inline))
			{
				if constexpr (!K_LDS) load_k(i);
#pragma unroll
				for (int nb = 0; nb < NB; ++nb)
#pragma unroll
					for (int mb = 0; mb < 2; ++mb)
					{
						f32x4 acc = c_init[nb];
#pragma unroll
						for (int kk = 0; kk < KK; ++kk)
						{
							bf16x8 a;
							if constexpr (K_LDS)
							{
								const int row = 16 * mb + col, slot = 4 * kk + grp;
								a = *reinterpret_cast<const bf16x8*>(kt + row * HD + 8 * (slot ^ kswz<HD>(row)));
							}
							else
								a = as_bf16x8(kreg[K_LDS ? 0 : mb][kk]);
							const bf16x8 qh = QHI_LDS ? *q_lds(1, nb, kk) : qhi[QHI_LDS ? 0 : nb][kk];
							acc = mfma16x16x32(a, qh, acc);
							acc = mfma16x16x32(a, *q_lds(0, nb, kk), acc);
						}
						sc[mb][nb] = acc;
					}
				if constexpr (K_LDS) load_k(i + 1); // past the last step: nothing in range, zeros
			};
			// Masks keys outside a row's span (only on steps that cross an edge)
			// and returns each row's maximum; true when some row's offset has to
			// grow (its scores exceed it by more than kLazy, or its first key).
			auto row_max = [&](int i, f32x4 (&sc)[2][NB], float (&mx)[NB]) __attribute__((always_inline)) -> bool
			{
				const int kw0 = kmin + i * kStep + wave * kWK;
				if (kw0 < first_hi || kw0 + kWK - 1 > last_lo)
				{
#pragma unroll
					for (int mb = 0; mb < 2; ++mb)
#pragma unroll
						for (int e = 0; e < 4; ++e)
						{
							const int k = kw0 + 16 * mb + 4 * grp + e;
#pragma unroll
							for (int nb = 0; nb < NB; ++nb)
								if (k < rfirst[nb] || k > rlast[nb]) sc[mb][nb][e] = -INFINITY;
						}
				}
				bool grow = false;
#pragma unroll
				for (int nb = 0; nb < NB; ++nb)
				{
					float m = fmaxf(fmaxf(fmaxf(sc[0][nb][0], sc[0][nb][1]), fmaxf(sc[0][nb][2], sc[0][nb][3])),
					                fmaxf(fmaxf(sc[1][nb][0], sc[1][nb][1]), fmaxf(sc[1][nb][2], sc[1][nb][3])));
					m = fmaxf(m, __shfl_xor(m, 16));
					m = fmaxf(m, __shfl_xor(m, 32));
					mx[nb] = m;
					grow |= m > kLazy || (m_off[nb] == -INFINITY && m != -INFINITY);
				}
				return __builtin_amdgcn_ballot_w64(grow) != 0;
			};
			// Raises the offsets that have to grow; rescales O, l and the scores.
			auto regrow = [&](f32x4 (&sc)[2][NB], const float (&mx)[NB]) __attribute__((always_inline))
			{
#pragma unroll
				for (int nb = 0; nb < NB; ++nb)
				{
					const bool fresh = m_off[nb] == -INFINITY;
					const bool g = mx[nb] > kLazy || (fresh && mx[nb] != -INFINITY);
					const float d = g ? mx[nb] : 0.0f;
					const float alpha = fresh ? 0.0f : fast_exp2(-d); // 1 when the row does not grow
					if (g) m_off[nb] = (fresh ? 0.0f : m_off[nb]) + d;
					const float ci = m_off[nb] == -INFINITY ? 0.0f : -m_off[nb];
					c_init[nb] = f32x4{ci, ci, ci, ci};
#pragma unroll
					for (int db = 0; db < DB; ++db) acc_o[db][nb] *= alpha;
					acc_l[nb] *= alpha;
#pragma unroll
					for (int mb = 0; mb < 2; ++mb) sc[mb][nb] -= d;
				}
			};
			// P^T (keys 16h + 4g + e in slot 8g + 4h + e) as the B operand of
			// O^T += V^T . P^T and of l += 1 . P^T; then step i + 1's V rows into
			// the tile, whose reads are done.
			auto accumulate = [&](int i, const f32x4 (&sc)[2][NB]) __attribute__((always_inline))
			{
				f16x8 pb[NB];
#pragma unroll
				for (int nb = 0; nb < NB; ++nb)
				{
					float w[8];
#pragma unroll
					for (int e = 0; e < 4; ++e)
					{
						w[e] = fast_exp2(sc[0][nb][e]);
						w[4 + e] = fast_exp2(sc[1][nb][e]);
					}
					pb[nb] = as_f16x8(u32x4{pack_f16x2(w[0], w[1]), pack_f16x2(w[2], w[3]), pack_f16x2(w[4], w[5]),
					                        pack_f16x2(w[6], w[7])});
				}
				// Lane (g, c) reads V^T for keys 16h + 4g + c / 4 (+0..3 across the
				// transpose) and elements 16 db + 4 (c % 4) .. + 4.
				const int trow = 4 * grp + (col >> 2);
#pragma unroll
				for (int db = 0; db < DB; ++db)
				{
					const int seg = 2 * db + ((col & 3) >> 1), half = 4 * (col & 1);
					const uint16_t* r0 = vt + trow * HD + 8 * (seg ^ vswz<HD>(trow)) + half;
					const uint16_t* r1 = vt + (trow + 16) * HD + 8 * (seg ^ vswz<HD>(trow + 16)) + half;
					const u32x2 lo = tr_read(r0);
					const u32x2 hi = tr_read(r1);
					const f16x8 a = as_f16x8(bf16x8_to_f16x8(u32x4{lo.x, lo.y, hi.x, hi.y}));
#pragma unroll
					for (int nb = 0; nb < NB; ++nb) acc_o[db][nb] = mfma16x16x32(a, pb[nb], acc_o[db][nb]);
				}
#pragma unroll
				for (int nb = 0; nb < NB; ++nb) acc_l[nb] = mfma16x16x32(ones, pb[nb], acc_l[nb]);
				load_v(i + 1); // past the last step: nothing in range, zeros
			};

			if (n_steps > 0)
			{
				if constexpr (K_LDS) load_k(0);
				load_v(0);
			}
			// The inner loop runs the steps that need no rescale; a step whose
			// scores outgrow a row's offset leaves it, is rescaled and finished
			// outside, so the O accumulators are only touched by MFMAs in the
			// common path.
			int i = 0;
			while (i < n_steps)
			{
				f32x4 sc[2][NB];
				float mx[NB];
				bool grow = false;
				for (; i < n_steps; ++i)
				{
					scores(i, sc);
					grow = row_max(i, sc, mx);
					if (grow) break;
					accumulate(i, sc);
				}
				if (!grow) break;
				regrow(sc, mx);
				accumulate(i, sc);
				++i;
			}

			// Merge the wavefronts: o = sum_w o_w 2^(m_w - M) / sum_w l_w 2^(m_w - M),
			// 0 when no key was seen (reference nn_ops.cpp:492).
			if (grp == 0)
			{
#pragma unroll
				for (int nb = 0; nb < NB; ++nb)
				{
					s_m[wave][16 * nb + col] = m_off[nb];
					s_l[wave][16 * nb + col] = acc_l[nb][0];
				}
			}
			__syncthreads(); // also: every V tile is done, s_raw becomes the merge buffer
			float* s_o = reinterpret_cast<float*>(s_raw);
#pragma unroll
			for (int nb = 0; nb < NB; ++nb)
			{
				const int r = 16 * nb + col;
				float M = s_m[0][r];
#pragma unroll
				for (int w = 1; w < kWaves; ++w) M = fmaxf(M, s_m[w][r]);
				float L = 0.0f, f_own = 0.0f;
#pragma unroll
				for (int w = 0; w < kWaves; ++w)
				{
					const float f = s_m[w][r] == -INFINITY ? 0.0f : fast_exp2(s_m[w][r] - M);
					L = fmaf(s_l[w][r], f, L);
					if (w == wave) f_own = f;
				}
				const float sc_own = L > 0.0f ? f_own / L : 0.0f;
				float* orow = s_o + (wave * ROWS + r) * OPITCH + 4 * grp;
#pragma unroll
				for (int db = 0; db < DB; ++db)
				{
					const f32x4 v = acc_o[db][nb] * sc_own;
					*reinterpret_cast<float4*>(orow + 16 * db) = make_float4(v[0], v[1], v[2], v[3]);
				}
			}
			__syncthreads();
			constexpr int Q4 = HD / 4; // float4s per row
			for (int idx = threadIdx.x; idx < ROWS * Q4; idx += 64 * kWaves)
			{
				const int r = idx / Q4, d4 = idx % Q4;
				const int gr = row0 + r;
				if (gr >= n_rows) continue;
				float4 acc = *reinterpret_cast<const float4*>(s_o + r * OPITCH + 4 * d4);
#pragma unroll
				for (int w = 1; w < kWaves; ++w)
				{
					const float4 v = *reinterpret_cast<const float4*>(s_o + (w * ROWS + r) * OPITCH + 4 * d4);
					acc.x += v.x;
					acc.y += v.y;
					acc.z += v.z;
					acc.w += v.w;
				}
				float* op = p.out + static_cast<size_t>(gr / G) * q_stride + static_cast<size_t>(kvh * G + gr % G) * HD;
				*reinterpret_cast<float4*>(op + 4 * d4) = acc;
			}
		}

		template <int HD>
		bool launch_hd(const prefill_params& p, int group, hipStream_t stream)
		{
			const dim3 grid(p.n_qtiles * p.n_kv), block(64 * kWaves);
			switch (group)
			{
			case 1: prefill_kernel<HD, 1><<<grid, block, 0, stream>>>(p); return true;
			case 2: prefill_kernel<HD, 2><<<grid, block, 0, stream>>>(p); return true;
			case 4: prefill_kernel<HD, 4><<<grid, block, 0, stream>>>(p); return true;
			case 8: prefill_kernel<HD, 8><<<grid, block, 0, stream>>>(p); return true;
			default: return false;
			}
		}
	}

	bool launch_prefill(prefill_params p, int head_dim, int group, bool bf16, hipStream_t stream)
	{
		if (!bf16) return false;
		const int rows = 16 * (head_dim == 64    ? prefill_cfg<64>::NB
		                       : head_dim == 128 ? prefill_cfg<128>::NB
		                                         : prefill_cfg<256>::NB);
		p.n_qtiles = (p.n_tok * group + rows - 1) / rows;
		switch (head_dim)
		{
		case 64: return launch_hd<64>(p, group, stream);
		case 128: return launch_hd<128>(p, group, stream);
		case 256: return launch_hd<256>(p, group, stream);
		default: return false;
		}
	}
}
