// Host-side declarations of the attention kernels' launchers and their
// parameter blocks. Shared by the bridge (nnc_hip.hip) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nnchip
{
	// Split-K attention of each query token independently (one token: the
	// decode step; several: the fp32-exact batch path) over one layer's K/V.
	struct decode_params
	{
		const float* q; // [n_tok][n_head * head_dim]
		float* out; // [n_tok][n_head * head_dim]
		const void* K; // [rows][kv_dim], BF16 bits or F32
		const void* V;
		const float* gate; // [n_tok][n_head * head_dim], or null: out *= sigmoid(gate) (Qwen3.5)
		float* part; // [n_tok][n_kv][n_split][group][head_dim + 4]: o, then m (log2 units), then l
		int rows, kv_dim, n_head, n_kv;
		int pos0, n_seq, window, causal; // token t sits at pos0 + t
		int n_tok; // tokens in this launch
		int split_base; // first key of split 0, a multiple of split_keys
		int split_keys; // keys per work-group, a multiple of decode_wg_keys()
		int n_split; // work-groups per (token, KV head), at most kDecodeMaxSplits
		float qscale; // scale * log2(e)
		// Per head group arrival counts for the fused merge (all zero
		// between launches), or null: then a separate merge launch follows.
		unsigned* counts;
	};

	constexpr int kDecodeMaxSplits = 256;

	// The fused merge: a one-token launch of the MFMA kernels over at most
	// kFuseMaxSplits splits merges inside the split launch. Each work-group
	// writes its partial device-coherently and counts itself in; the last of
	// a head group to arrive merges the group's splits with the operations of
	// the merge kernel, so the bits do not depend on which path ran. The
	// short spans of decode (a sliding window, a small context) are where a
	// second launch costs as much as the split itself.
	constexpr int kFuseMaxSplits = 8, kFuseCounts = 4096;
	__host__ __device__ inline bool fused_merge_on(const decode_params& p)
	{
		return p.counts != nullptr && p.n_tok == 1 && p.n_split > 1 && p.n_split <= kFuseMaxSplits;
	}

	// KV heads per work-group of the BF16 kernels: two when n_kv is even (a
	// work-group then reads runs of 2 * head_dim elements of each row, two
	// wavefronts per head), else one (four wavefronts per head). Every BF16
	// kernel splits a head's keys among its wavefronts the same way, which is
	// what keeps a token's bits independent of the kernel that computes it.
	inline int bf16_heads_per_wg(int n_kv) { return n_kv % 2 == 0 ? 2 : 1; }

	// The head shapes of the MFMA kernels: head_dim 64, 128 or 256 with 1, 2,
	// 4 or 8 query heads per KV head. Every other shape nnc runs (an even
	// head_dim up to 512, group * head_dim up to kGenMaxGroupDim) takes the
	// generic split-K kernels, for every batch size.
	constexpr int kGenMaxGroup = 16, kGenMaxGroupDim = 8192;
	__host__ __device__ inline bool mfma_shape(int head_dim, int group)
	{
		return (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
		       (group == 1 || group == 2 || group == 4 || group == 8);
	}
	__host__ __device__ inline bool generic_shape_ok(int head_dim, int group)
	{
		return head_dim > 0 && head_dim % 2 == 0 && head_dim <= 512 && group >= 1 && group <= kGenMaxGroup &&
		       group * head_dim <= kGenMaxGroupDim;
	}

	// Work-groups per split (head groups) and the keys one work-group
	// consumes per iteration, for a head shape, element type and n_kv;
	// split_keys must be a multiple of the latter (256, nnc's block, for the
	// generic kernels).
	int decode_groups(int n_kv, bool bf16, int head_dim, int group);
	int decode_wg_keys(int head_dim, int group, bool bf16, int n_kv);
	// Keys of one wavefront chunk: a split may be any multiple of it (a
	// split shorter than decode_wg_keys leaves some wavefronts without a
	// chunk).
	int decode_chunk_keys(int head_dim, int group, bool bf16);

	// Launches the decode kernel over an (n_split, head groups, token groups)
	// grid, then (n_split > 1) the split merge over (n_kv * group * slices, n_tok);
	// returns false when (head_dim, group, bf16) has no instantiation. A
	// token's result depends only on its own span and the split grid
	// (split_keys and the absolute split boundaries), not on the other tokens
	// of the launch.
	bool launch_decode(const decode_params& p, int n_tok, int head_dim, int group, bool bf16, hipStream_t stream);

	// The generic split-K kernels (and their ordered merge) for a shape
	// outside mfma_shape; false when generic_shape_ok fails.
	bool launch_decode_generic(const decode_params& p, int n_tok, int head_dim, int group, bool bf16,
	                           hipStream_t stream);

	// The ordered merge of the generic kernels' split partials (n_split > 1)
	// over an (n_kv * group, n_tok) grid; writes o * (1 / l).
	void launch_merge_generic(const decode_params& p, int n_tok, int head_dim, int group, hipStream_t stream);

	// The tiled fp32-MFMA kernel for batches of F32 caches and of head shapes
	// outside mfma_shape: head_dim a multiple of 16 up to 512, group up to 16.
	// Grid (row blocks of 64, n_kv, n_split) over the absolute split grid of
	// p.split_keys (a multiple of 16) keys, then (n_split > 1) the generic
	// merge; false when tiled_shape_ok fails.
	__host__ __device__ inline bool tiled_shape_ok(int head_dim, int group)
	{
		return head_dim > 0 && head_dim % 16 == 0 && head_dim <= 512 && group >= 1 && group <= kGenMaxGroup;
	}
	bool launch_tiled(const decode_params& p, int n_tok, int head_dim, int group, bool bf16, hipStream_t stream);

	// Tiled MFMA attention for a batch of query tokens.
	struct prefill_params
	{
		const float* q; // [n_tok][n_head * head_dim]
		float* out; // [n_tok][n_head * head_dim]
		const float* gate; // [n_tok][n_head * head_dim], or null: out *= sigmoid(gate) (Qwen3.5)
		const void* K; // [rows][kv_dim]
		const void* V;
		const void* V16; // fp16 copy of V (blocked: f16_copy_index), or null
		const int* n_bad; // elements of the copy marked kF16Bad (beyond kF16CopyMax); not 0: use V
		int rows, kv_dim, n_head, n_kv;
		int n_tok, pos0, n_seq, window;
		int causal;
		int n_qtiles; // query tiles per KV head (set by launch_prefill)
		float qscale; // scale * log2(e)
	};

	bool launch_prefill(prefill_params p, int head_dim, int group, bool bf16, hipStream_t stream);

	// Bytes of a buffer's fp16 copy of V: its rows rounded up to whole groups
	// of 32 (the copy's blocked layout, f16_copy_index in device_common.h).
	inline size_t f16_copy_bytes(int rows, int kv_dim)
	{
		return static_cast<size_t>((rows + 31) / 32) * 32 * static_cast<size_t>(kv_dim) * 2;
	}

	// F32 rows -> the cache's element type, row (pos0 + t) % rows.
	constexpr int kPrepMaxPairs = 256; // RoPE pairs per head (head_dim up to 512)

	// The pre-attention step of one batch (reference model.cpp:1616-1691).
	struct prep_params
	{
		float* q; // [n_tok][n_head * head_dim], normalised and rotated in place
		const float* k; // [n_tok][kv_dim]
		const float* v; // [n_tok][kv_dim]
		void* K; // the layer's buffers: [rows][kv_dim], BF16 bits or F32
		void* V;
		void* V16; // V's fp16 copy (BF16 buffers), or null
		int* n_bad; // the copy's count of kF16Bad elements
		const float* q_gamma; // head_dim floats, or null: no Q norm
		const float* k_gamma; // head_dim floats, or null: no K norm
		// cos and sin of every rotation angle of the batch, [n_tok][n_rot / 2]
		// (cos, sin) pairs, computed on the host as the reference computes them
		const float2* rope_cs;
		int n_head, n_kv, head_dim, rows, pos0, bf16;
		int v_norm; // RMS-normalise V per head, no gamma
		int n_rot; // rotated lanes per head (even); 0: no RoPE
		int mode; // 0 NEOX, 1 NORM
		float eps;
		float inv_dim; // 1 / head_dim in fp32 (the gamma norm's mean)
	};

	// Launches the pre-attention step over an (n_head + 2 n_kv, n_tok) grid of
	// head rows; false for a head_dim or n_rot outside the supported range.
	bool launch_prep(const prep_params& p, int n_tok, hipStream_t stream);

	// V16, n_bad: the buffer's fp16 copy of V and its count of kF16Bad
	// elements (values beyond kF16CopyMax; kept up to date as elements are
	// replaced), or null (no copy).
	bool launch_append_f32(void* K, void* V, const float* k_rows, const float* v_rows, int rows, int kv_dim, int pos0,
	                       int n_tok, bool bf16, hipStream_t stream, void* V16, int* n_bad);

	// The fp16 copy of BF16 V rows pos0 .. pos0 + n_tok - 1 (mod rows).
	bool launch_shadow_rows(const void* V, void* V16, int* n_bad, int rows, int kv_dim, int pos0, int n_tok,
	                        hipStream_t stream);

	bool launch_fill_normal(void* dst, uint64_t n, uint64_t seed, int norm_dim, bool bf16, hipStream_t stream);

	// The weight gemvs (reference nn_ops.h:95-180): Y[t] = W . X[t] for
	// t < n_batch <= 16, W in one of nnc's three weight layouts.
	constexpr int kGemvBf16 = 0, kGemvQ8_0 = 1, kGemvQ4S = 2;
	constexpr int kGemvMaxBatch = 16;
	constexpr size_t kGemvLdsBudget = 64 << 10; // dynamic LDS per one-vector gemv work-group
	// The batch kernel: weight rows per work-group (16 per wavefront) and its
	// dynamic LDS budget per weight layout (at most two work-groups per CU),
	// which sets the K splits. Measured against 64 rows and 64 KiB (a 16-vector
	// Qwen3-4B layer, us): BF16 94.4 -> 91.6 (80 KiB; 98.0 at 64, 93.3 at 96),
	// Q8_0 114.2 -> 97.0 and Q4_S 122.1 -> 96.6 (48 KiB; at 32 / 40 / 56 / 64 /
	// 80 KiB Q8_0 107.1 / 98.4 / 107.4 / 105.6 / 105.5, Q4_S 105.3 / 102.4 /
	// 106.9 / 105.0 / 110.6: the quantised kernels, slower per byte, gain from
	// the work-groups of more splits); the X^T staged per weight byte halves.
	constexpr int kGemvRows = 128;
	constexpr size_t gemv_batch_lds(int format) { return format == kGemvBf16 ? 80 << 10 : 48 << 10; }

	// LDS of a gemv work-group over `blocks` 32-column blocks and n_batch
	// tokens: X^T hi and lo (bf16), the kGemvRows rows' scales and biases, and
	// the Q4_S block sums.
	__host__ __device__ inline size_t gemv_lds_bytes(int blocks, int n_batch)
	{
		return static_cast<size_t>(blocks) * (128 * n_batch + 4 * kGemvRows + 4 * n_batch);
	}

	// One weight matrix of a gemv: its rows' weights, scales and biases, and
	// where its outputs go.
	struct gemv_mat
	{
		const void* w; // BF16 [rows][cols], Q8_0 int8 [rows][cols], Q4_S nibbles [rows][cols / 2]
		const uint16_t* scales; // [rows][cols / 32] BF16 (Q8_0, Q4_S)
		const uint16_t* biases; // [rows][cols / 32] BF16 (Q4_S)
		float* y; // [n_batch] vectors of rows floats, y_stride apart
		size_t y_stride;
	};

	// Matrices sharing X in one launch, stacked along the rows.
	constexpr int kGemvMaxMats = 3;

	struct gemv_params
	{
		int format; // kGemvBf16, kGemvQ8_0 or kGemvQ4S
		// Matrix m holds stacked rows mrow[m] .. mrow[m + 1] - 1 (mrow[0] = 0,
		// mrow[n_mat] = rows, later entries INT_MAX). Every matrix but the last
		// has a multiple of 16 rows, so no row pair of the one-vector kernel
		// and no 16-row tile of the batch kernel spans two matrices.
		gemv_mat mats[kGemvMaxMats];
		int mrow[kGemvMaxMats + 1];
		const float* x; // [n_batch] vectors of cols floats, x_stride apart
		const float* xsum; // Q4_S: [n_batch] runs of cols / 32 block sums, xsum_stride apart; or null
		float* part; // [n_split][n_batch][rows] partial sums when n_split > 1 (stacked rows)
		size_t x_stride, xsum_stride;
		int rows, cols, n_batch; // rows: all matrices' rows
		int n_split, split_blocks; // K splits, and 32-column blocks per split
		// argmax of y instead of y (BF16, one vector): each work-group's best
		// (value, row) pair, then the row
		float2* best; // [work-groups] (value, row as int bits; row -1 when none)
		int* argmax; // the result, then whether y[0] is NaN
		int first_sticks; // 1: the result is 0 when y[0] is NaN (the reference's linear scan from y[0])
	};

	// K splits for a (rows, cols) gemv of n_batch vectors.
	void gemv_plan(int rows, int cols, int n_batch, int format, int& n_split, int& split_blocks);

	bool launch_gemv(const gemv_params& p, hipStream_t stream);

	// Work-groups of the one-vector kernel for `rows` rows (the number of
	// best pairs launch_gemv_argmax writes), and whether a gemv of `cols`
	// columns and n_batch vectors runs on it.
	int gemv_vec_groups(int rows);
	bool gemv_vec_fits(int cols, int n_batch, int format);

	// argmax_r y[r] for a BF16 gemv of one vector (p.best, p.argmax set):
	// the smallest row of the largest value above -inf, NaN never chosen, 0
	// when there is none. Needs gemv_vec_fits(p.cols, 1, kGemvBf16).
	bool launch_gemv_argmax(const gemv_params& p, hipStream_t stream);

	// The same argmax over a float vector y of p.rows elements (p.y read, p.best
	// and p.argmax set; at most kArgmaxGroups pairs).
	constexpr int kArgmaxGroups = 512;
	bool launch_argmax(const gemv_params& p, hipStream_t stream);

	bool launch_zero(float* dst, size_t n, hipStream_t stream);

	// n floats from src (device memory or pinned host memory, 16-byte
	// aligned) to dst (device memory), on the stream.
	bool launch_copy(float* dst, const float* src, size_t n, hipStream_t stream);

	// The span of keys position `pos` attends to (reference model.cpp:2300-2316).
	__host__ __device__ inline void attn_span(int causal, int window, int pos, int n_seq, int& first, int& last)
	{
		if (causal)
		{
			first = (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
			last = pos < n_seq - 1 ? pos : n_seq - 1;
		}
		else if (window > 0)
		{
			first = pos - window / 2 > 0 ? pos - window / 2 : 0;
			last = pos + window / 2 < n_seq - 1 ? pos + window / 2 : n_seq - 1;
		}
		else
		{
			first = 0;
			last = n_seq - 1;
		}
	}
}
