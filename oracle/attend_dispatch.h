// TEST INFRASTRUCTURE — part of the CPU oracle. Only tests/, the smoke check
// and bench.py's cpu_baseline leg may load code built from this file; the
// product path never does.
//
// Layer-granularity attention over nnc's K/V layout: for every query token t
// of a batch at positions pos0 + t, and every KV head, the keys of t's span
// are cut into 256-key blocks aligned to absolute positions, each block gives
// a partial (o, m, l) per query head of the group, and the partials are merged
// in block order. This restates nnc's attention core:
//   - attn_job / attend_block / attend_token / attend_chunks / attend_blocks
//     (reference src/libnnc/model.cpp:1229-1317);
//   - the byte count, the 256 KiB parallel threshold, the three paths and the
//     decode merge in block order (reference src/libnnc/model.cpp:1707-1757);
//   - slots = max(1, min(threads, 64)) (reference src/libnnc/model.cpp:1977).
// The kernels (block / merge / finish) and the thread pool come in through an
// `Ops` policy, so the same dispatch drives both this repository's own
// restatement of the kernels and the reference's compiled ones.
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <vector>

namespace orc
{
	constexpr int kAttnBlock = 256; // keys per block (reference model.h:229)
	constexpr uint64_t kParallelBytes = 256u << 10; // reference model.cpp:1730

	inline size_t part_floats(size_t head_dim) { return head_dim + 2; } // reference nn_ops.h:45

	// One layer's attention call, in the units the op works in.
	struct attend_args
	{
		const float* q; // [n_tok][n_head * head_dim]
		float* out; // [n_tok][n_head * head_dim]
		const uint8_t* K; // [rows][n_kv * head_dim] of BF16 (uint16) or F32
		const uint8_t* V;
		bool kv_bf16;
		int rows;
		int n_tok, pos0, n_seq, window;
		bool causal;
		int n_head, n_kv, head_dim;
		float scale;
	};

	// The span of keys position `pos` attends to (reference model.cpp:2300-2316).
	inline void attn_span(bool causal, int window, int pos, int n_seq, int* first, int* last)
	{
		if (causal)
		{
			*first = (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
			*last = std::min(pos, n_seq - 1);
			return;
		}
		if (window > 0)
		{
			*first = std::max(0, pos - window / 2);
			*last = std::min(n_seq - 1, pos + window / 2);
			return;
		}
		*first = 0;
		*last = n_seq - 1;
	}

	// Scores slots and decode partials, kept across calls so that a timed call
	// allocates nothing once warm (the reference sizes them once, in
	// model_kv_init, reference model.cpp:1970-1980).
	struct attend_scratch
	{
		std::vector<float> slots, parts;
		static void reserve(std::vector<float>& v, size_t n)
		{
			if (v.size() < n) v.resize(n);
		}
	};

	template <class Ops>
	class attend_runner
	{
	public:
		attend_runner(const Ops& ops, const attend_args& a, attend_scratch& s) : ops_(ops), a_(a), s_(s)
		{
			group_ = a.n_head / a.n_kv;
			hd_ = static_cast<size_t>(a.head_dim);
			kv_dim_ = static_cast<size_t>(a.n_kv) * hd_;
			esize_ = a.kv_bf16 ? 2 : 4;
			part_ = static_cast<size_t>(group_) * part_floats(hd_);
			// A slot: scores of every head of the group over one block, then
			// two partials (reference model.cpp:1975-1978).
			slot_ = static_cast<size_t>(group_) * kAttnBlock + 2 * part_;
			n_slots_ = std::max(1, std::min(ops_.n_threads(), 64));
		}

		void run()
		{
			const attend_args& a = a_;
			uint64_t bytes = 0;
			for (int t = 0; t < a.n_tok; ++t)
			{
				int first, last;
				attn_span(a.causal, a.window, a.pos0 + t, a.n_seq, &first, &last);
				bytes += 2ull * static_cast<uint64_t>(last + 1 - first) * kv_dim_ * esize_;
			}
			if (a.n_tok == 1 && bytes >= kParallelBytes && n_slots_ > 1)
			{
				// Decode: (KV head, block) items shared out, merged in block order.
				int first, last;
				attn_span(a.causal, a.window, a.pos0, a.n_seq, &first, &last);
				blk0_ = first / kAttnBlock;
				n_blk_ = last / kAttnBlock + 1 - blk0_;
				const int n_items = a.n_kv * n_blk_;
				n_chunks_ = std::min(n_items, n_slots_);
				attend_scratch::reserve(s_.slots, slot_ * n_chunks_);
				attend_scratch::reserve(s_.parts, part_ * static_cast<size_t>(n_items));
				ops_.parallel_for(static_cast<uint32_t>(n_chunks_), &attend_runner::blocks_range, this);
				for (int kvh = 0; kvh < a.n_kv; ++kvh)
				{
					float* acc = s_.parts.data() + static_cast<size_t>(kvh) * n_blk_ * part_;
					for (int b = 1; b < n_blk_; ++b) ops_.merge(acc, acc + b * part_, hd_, group_);
					ops_.finish(a.out + static_cast<size_t>(kvh) * group_ * hd_, hd_, acc, hd_, group_);
				}
				return;
			}
			n_chunks_ = std::min(a.n_tok, n_slots_);
			if (n_chunks_ > 1 && bytes >= kParallelBytes)
			{
				attend_scratch::reserve(s_.slots, slot_ * n_chunks_);
				ops_.parallel_for(static_cast<uint32_t>(n_chunks_), &attend_runner::chunks_range, this);
			}
			else
			{
				attend_scratch::reserve(s_.slots, slot_);
				for (int t = 0; t < a.n_tok; ++t) token(t, s_.slots.data());
			}
		}

	private:
		// Partial of token t's group on KV head kvh over the part of
		// [first, last] in block b (reference model.cpp:1249-1263).
		void block(int t, int kvh, int first, int last, int b, float* scores, float* part) const
		{
			const attend_args& a = a_;
			const int k0 = std::max(first, b * kAttnBlock);
			const int k1 = std::min(last, b * kAttnBlock + kAttnBlock - 1);
			const size_t off = (static_cast<size_t>(k0 % a.rows) * kv_dim_ + static_cast<size_t>(kvh) * hd_) * esize_;
			const float* qh = a.q + static_cast<size_t>(t) * a.n_head * hd_ + static_cast<size_t>(kvh) * group_ * hd_;
			ops_.block(qh, hd_, a.K + off, a.V + off, a.kv_bf16, kv_dim_, static_cast<size_t>(k1 + 1 - k0), hd_,
			           static_cast<size_t>(group_), a.scale, scores, part);
		}

		// Every KV head of token t, blocks merged in order (reference model.cpp:1265-1291).
		void token(int t, float* slot) const
		{
			const attend_args& a = a_;
			int first, last;
			attn_span(a.causal, a.window, a.pos0 + t, a.n_seq, &first, &last);
			float* scores = slot;
			float* acc = slot + static_cast<size_t>(group_) * kAttnBlock;
			float* tmp = acc + part_;
			float* out_t = a.out + static_cast<size_t>(t) * a.n_head * hd_;
			const int b0 = first / kAttnBlock, b1 = last / kAttnBlock;
			for (int kvh = 0; kvh < a.n_kv; ++kvh)
			{
				block(t, kvh, first, last, b0, scores, acc);
				for (int b = b0 + 1; b <= b1; ++b)
				{
					block(t, kvh, first, last, b, scores, tmp);
					ops_.merge(acc, tmp, hd_, group_);
				}
				ops_.finish(out_t + static_cast<size_t>(kvh) * group_ * hd_, hd_, acc, hd_, group_);
			}
		}

		// Chunk c: tokens c, c + n_chunks, ... (reference model.cpp:1293-1301).
		static void chunks_range(uint32_t c0, uint32_t c1, void* user)
		{
			const auto& self = *static_cast<const attend_runner*>(user);
			for (uint32_t c = c0; c < c1; ++c)
				for (int t = static_cast<int>(c); t < self.a_.n_tok; t += self.n_chunks_)
					self.token(t, self.s_.slots.data() + c * self.slot_);
		}

		// Decode chunk c: items c, c + n_chunks, ... of (KV head, block), each
		// into its own partial (reference model.cpp:1303-1317).
		static void blocks_range(uint32_t c0, uint32_t c1, void* user)
		{
			const auto& self = *static_cast<const attend_runner*>(user);
			const attend_args& a = self.a_;
			int first, last;
			attn_span(a.causal, a.window, a.pos0, a.n_seq, &first, &last);
			const int n_items = a.n_kv * self.n_blk_;
			float* scratch = self.s_.slots.data();
			float* parts = self.s_.parts.data();
			for (uint32_t c = c0; c < c1; ++c)
				for (int i = static_cast<int>(c); i < n_items; i += self.n_chunks_)
					self.block(0, i / self.n_blk_, first, last, self.blk0_ + i % self.n_blk_, scratch + c * self.slot_,
					           parts + static_cast<size_t>(i) * self.part_);
		}

		const Ops& ops_;
		const attend_args& a_;
		attend_scratch& s_;
		int group_ = 1;
		size_t hd_ = 0, kv_dim_ = 0, esize_ = 4, part_ = 0, slot_ = 0;
		int n_slots_ = 1, n_chunks_ = 1, blk0_ = 0, n_blk_ = 0;
	};

	// K/V rows of a buffer: a causal sliding layer keeps a ring of
	// round_up(window + n_batch, 256) rows when that is smaller than the
	// context, else n_ctx rows (reference model.cpp:1936-1957).
	inline int kv_rows(int n_ctx, int window, int n_batch)
	{
		const int nb = n_batch > 0 ? n_batch : 1;
		const int ring = (window + nb + kAttnBlock - 1) / kAttnBlock * kAttnBlock;
		return (window > 0 && ring < n_ctx) ? ring : n_ctx;
	}
}
