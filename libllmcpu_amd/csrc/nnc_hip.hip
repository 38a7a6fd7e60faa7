// The C-ABI bridge declared in include/nnc_hip.h: device K/V buffers that
// mirror model_kv_init's (reference src/libnnc/model.cpp:1891-1957), the
// append of reference model.cpp:1662-1691, and one attention call per layer
// in place of the attention core of reference model.cpp:1693-1761.
//
// Every entry point checks its arguments before touching the device, so a
// refused call changes nothing (the "fail before it changes anything" rule of
// reference model.cpp:2046-2057). Failures set a thread-local message and
// return an nnc_status; no C++ exception crosses the ABI.
#include "../../include/nnc_hip.h"
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

// The decode partials of nnc_hip_attend_device_noalloc: a fixed array in
// every device's global memory, held until the process ends. In host code
// this name is only a stand-in for the symbol; its device address comes from
// hipGetSymbolAddress, once per device (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[NNC_HIP_NOALLOC_SCRATCH_BYTES];

namespace
{
	thread_local std::string g_last_error = "";

	// The log callback (nnc's own, in a drop-in build) and its user pointer;
	// none: warnings and errors go to stderr, as nnc's default does.
	std::mutex g_log_mu;
	nnc_hip_log_callback g_log_cb = nullptr;
	void* g_log_user = nullptr;

	void log_msg(int level, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

	void log_msg(int level, const char* fmt, ...)
	{
		char buf[512];
		va_list ap;
		va_start(ap, fmt);
		std::vsnprintf(buf, sizeof buf, fmt, ap);
		va_end(ap);
		std::lock_guard<std::mutex> lock(g_log_mu);
		if (g_log_cb)
			g_log_cb(level, buf, g_log_user);
		else if (level >= NNC_HIP_LOG_WARN)
			std::fprintf(stderr, "nnc_hip: %s\n", buf);
	}

	nnc_status fail(nnc_status status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

	nnc_status fail(nnc_status status, const char* fmt, ...)
	{
		char buf[512];
		va_list ap;
		va_start(ap, fmt);
		std::vsnprintf(buf, sizeof buf, fmt, ap);
		va_end(ap);
		g_last_error = buf;
		return status;
	}

	// A device runtime failure. Out-of-memory maps to nnc's own status; any
	// other fault of the device runtime is reported as an I/O failure of the
	// device, with the runtime's text.
	nnc_status hip_fail(hipError_t e, const char* what)
	{
		if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
			return fail(NNC_ERR_OUT_OF_MEMORY, "%s: device out of memory", what);
		return fail(NNC_ERR_IO, "%s: %s", what, hipGetErrorString(e));
	}

#define NNC_HIP_TRY(expr, what)                                                                                     \
	do                                                                                                                \
	{                                                                                                                 \
		const hipError_t e_ = (expr);                                                                                 \
		if (e_ != hipSuccess) return hip_fail(e_, what);                                                             \
	} while (0)

	// V starts kVOffset bytes into its allocation, so a K row and its V row
	// do not start on the same HBM channel. Measured on Qwen3-4B decode at
	// 32 768 keys (one box, fresh processes): 28.83 us per layer with K and V
	// aligned alike, 28.55 with V 256 bytes in, 28.75 with 512, 28.54 with
	// 768; a bare stream of the same head slices: the slices at bytes 256 and
	// 1280 of each row finish 15 % after the others when aligned alike.
	constexpr size_t kVOffset = 256;

	struct kv_buffer
	{
		void* k = nullptr;
		void* v = nullptr; // v_alloc + kVOffset
		// BF16 caches: an fp16 copy of v for the prefill kernel, kept by every
		// append (its P . V products then take P in fp16, one MFMA each); null
		// when disabled (NNC_HIP_F16_SHADOW=0). v16_alloc + kVOffset.
		void* v16 = nullptr;
		void* v_alloc = nullptr;
		void* v16_alloc = nullptr;
		int32_t rows = 0;
		int32_t kv_dim = 0;
	};

	// Grow-only device scratch.
	struct dev_scratch
	{
		void* ptr = nullptr;
		size_t bytes = 0;
	};

	// Pinned host memory (hipHostMalloc, coherent) through which the
	// host-buffer entry points move rows: appended rows and RoPE tables go to
	// the device by DMA, q is read once by a copy kernel, and the kernels
	// write out straight into it, so the caller's buffers are free on return.
	// `free` is recorded after the last device access of the buffer; the host
	// waits on it before writing again.
	struct host_staging
	{
		void* ptr = nullptr;
		size_t bytes = 0;
		hipEvent_t free = nullptr;
	};

	// One table of RoPE cos/sin pairs on the device ([n_tok][n_rot / 2]) and
	// what it was computed for; a model's layers share positions and usually
	// one rotation setup, so most calls find their table already there.
	struct rope_table
	{
		int32_t pos0 = -1, n_tok = 0, n_rot = 0;
		float base = 0.0f, pos_scale = 0.0f;
		bool has_ff = false;
		std::vector<float> ff;
		dev_scratch dev;
		uint64_t used = 0; // last use (for replacing the older table)
	};

	// Where a call's decode partials go: a fixed array of `bytes` bytes, or
	// (ptr null) the cache's grow-only scratch.
	struct part_source
	{
		float* ptr = nullptr;
		size_t bytes = 0;
	};

	// The device address of `scratch` on each device, looked up on the
	// device's first no-alloc call with that device current.
	constexpr int kMaxDevices = 64;
	std::mutex g_scratch_mu;
	void* g_scratch_ptr[kMaxDevices] = {};

	constexpr int32_t kDecodeChunk = 1024; // tokens per split-K launch
	constexpr int32_t kTiledChunk = 2048; // tokens per tiled launch (rows / 64 blocks on the grid's x)
	// Most tokens one forward pass of an nnc session carries
	// (MODEL_PREFILL_BATCH, reference model.h:330; session.cpp:340), its MTP
	// verification batches included (n_draft + 1, session.cpp:357, :516).
	// Batches up to this size run through the split-K kernel on each token's
	// own split grid, so every token gets the bits a one-token call gives it.
	constexpr int32_t kSessionBatch = 16;

	// NNC_HIP_F16_SHADOW=0 keeps no fp16 copy of BF16 caches (half the device
	// memory; the prefill kernel then converts V and splits Q on the fly).
	bool f16_shadow_enabled()
	{
		const char* e = std::getenv("NNC_HIP_F16_SHADOW");
		return !(e && e[0] == '0');
	}
}

struct nnc_hip_kv
{
	int device = 0;
	int n_cu = 256;
	bool bf16 = true;
	bool exact_batches = false; // batches over kSessionBatch tokens on the split-K path too
	hipStream_t stream = nullptr;
	std::vector<kv_buffer> bufs;
	uint64_t bytes = 0;
	dev_scratch part; // decode partials
	dev_scratch q; // device copies of host q / gate and append rows
	dev_scratch gate;
	dev_scratch gemv_part; // weight gemv partial sums over K splits
	int* n_bad = nullptr; // per buffer: elements of V's fp16 copy now marked kF16Bad (device)
	unsigned* counts = nullptr; // kFuseCounts arrival counts of the fused decode merge (device, zero between calls)
	dev_scratch rows_k;
	dev_scratch rows_v;
	host_staging pinned; // host rows in and out (q, gate, out; K/V appends; RoPE tables)
	rope_table rope[2]; // the last two RoPE setups (Gemma 3 alternates local and global layers)
	uint64_t rope_clock = 0;
};

namespace
{
	void release(nnc_hip_kv* kv)
	{
		if (!kv) return;
		if (kv->stream) (void)hipStreamSynchronize(kv->stream);
		for (auto& b : kv->bufs)
		{
			for (void* ptr : {b.k, b.v_alloc, b.v16_alloc})
				if (ptr) (void)hipFree(ptr);
		}
		if (kv->n_bad) (void)hipFree(kv->n_bad);
		if (kv->counts) (void)hipFree(kv->counts);
		for (dev_scratch* s : {&kv->part, &kv->q, &kv->gate, &kv->gemv_part, &kv->rows_k, &kv->rows_v,
		                       &kv->rope[0].dev, &kv->rope[1].dev})
			if (s->ptr) (void)hipFree(s->ptr);
		if (kv->pinned.ptr) (void)hipHostFree(kv->pinned.ptr);
		if (kv->pinned.free) (void)hipEventDestroy(kv->pinned.free);
		if (kv->stream) (void)hipStreamDestroy(kv->stream);
		delete kv;
	}

	// Makes s at least `bytes` long; the old allocation is freed after the
	// stream has drained.
	nnc_status reserve(nnc_hip_kv* kv, dev_scratch& s, size_t bytes, const char* what)
	{
		if (s.bytes >= bytes) return NNC_OK;
		NNC_HIP_TRY(hipStreamSynchronize(kv->stream), what);
		if (s.ptr) NNC_HIP_TRY(hipFree(s.ptr), what);
		s.ptr = nullptr;
		s.bytes = 0;
		const size_t n = (std::max<size_t>(bytes, 256) + 255) & ~static_cast<size_t>(255);
		NNC_HIP_TRY(hipMalloc(&s.ptr, n), what);
		s.bytes = n;
		return NNC_OK;
	}

	// Makes the pinned staging at least `bytes` long and free to write (every
	// earlier copy out of it has completed).
	nnc_status reserve_pinned(nnc_hip_kv* kv, size_t bytes, const char* what)
	{
		host_staging& h = kv->pinned;
		if (h.free) NNC_HIP_TRY(hipEventSynchronize(h.free), what);
		if (h.bytes >= bytes) return NNC_OK;
		if (h.ptr) NNC_HIP_TRY(hipHostFree(h.ptr), what);
		h.ptr = nullptr;
		h.bytes = 0;
		const size_t n = (std::max<size_t>(bytes, 64 << 10) + 4095) & ~static_cast<size_t>(4095);
		NNC_HIP_TRY(hipHostMalloc(&h.ptr, n, hipHostMallocCoherent), what);
		h.bytes = n;
		return NNC_OK;
	}


	// The cos/sin of every RoPE angle of tokens pos0 .. pos0 + n_tok - 1 on the
	// device, computed on the host the way the reference computes them
	// (nn_ops.cpp:1840-1855, model.cpp:1645-1655): the position (pos0 + t) *
	// pos_scale in fp32, the frequency ratio base^(-2/n_rot) with powf and the
	// per-pair frequency multiplied in step by step in fp32, the angle
	// position * frequency divided by the pair's frequency factor, and its cos
	// and sin from the host's libm (sincosf, whose results equal glibc's cosf
	// and sinf). The host's libm is the one nnc's own CPU path calls in the
	// same process, so the bits agree. Kept for the next call with the same
	// setup; the upload goes through the pinned staging on the cache's stream.
	nnc_status rope_cs(nnc_hip_kv* kv, const nnc_hip_prep& pr, int32_t pos0, int32_t n_tok, const float2*& out)
	{
		const int half = pr.n_rot / 2;
		auto same = [&](const rope_table& r)
		{
			if (r.pos0 != pos0 || r.n_tok != n_tok || r.n_rot != pr.n_rot) return false;
			if (std::memcmp(&r.base, &pr.freq_base, 4) != 0 || std::memcmp(&r.pos_scale, &pr.pos_scale, 4) != 0)
				return false;
			if (r.has_ff != (pr.freq_factors != nullptr)) return false;
			return !r.has_ff || std::memcmp(r.ff.data(), pr.freq_factors, sizeof(float) * half) == 0;
		};
		rope_table* hit = nullptr;
		for (rope_table& r : kv->rope)
			if (same(r)) hit = &r;
		if (!hit)
		{
			hit = kv->rope[0].used <= kv->rope[1].used ? &kv->rope[0] : &kv->rope[1];
			const size_t bytes = sizeof(float2) * static_cast<size_t>(n_tok) * half;
			hit->pos0 = -1; // (invalid until filled)
			if (nnc_status s = reserve(kv, hit->dev, bytes, "RoPE table")) return s;
			if (nnc_status s = reserve_pinned(kv, bytes, "RoPE table staging")) return s;
			float2* cs = static_cast<float2*>(kv->pinned.ptr);
			const float ratio = std::pow(pr.freq_base, -2.0f / static_cast<float>(pr.n_rot));
			std::vector<float> inv(half);
			float f = 1.0f;
			for (int i = 0; i < half; ++i)
			{
				inv[i] = f;
				f *= ratio;
			}
			for (int32_t t = 0; t < n_tok; ++t)
			{
				const float rpos = static_cast<float>(pos0 + t) * pr.pos_scale;
				for (int i = 0; i < half; ++i)
				{
					float th = rpos * inv[i];
					if (pr.freq_factors) th /= pr.freq_factors[i];
					float s, c;
					::sincosf(th, &s, &c);
					cs[static_cast<size_t>(t) * half + i] = make_float2(c, s);
				}
			}
			NNC_HIP_TRY(hipMemcpyAsync(hit->dev.ptr, cs, bytes, hipMemcpyHostToDevice, kv->stream), "RoPE table");
			NNC_HIP_TRY(hipEventRecord(kv->pinned.free, kv->stream), "RoPE table");
			hit->pos0 = pos0;
			hit->n_tok = n_tok;
			hit->n_rot = pr.n_rot;
			hit->base = pr.freq_base;
			hit->pos_scale = pr.pos_scale;
			hit->has_ff = pr.freq_factors != nullptr;
			hit->ff.assign(pr.freq_factors ? pr.freq_factors : nullptr, pr.freq_factors ? pr.freq_factors + half : nullptr);
		}
		hit->used = ++kv->rope_clock;
		out = static_cast<const float2*>(hit->dev.ptr);
		return NNC_OK;
	}

	nnc_status check_kv(const nnc_hip_kv* kv, int32_t buf)
	{
		if (!kv) return fail(NNC_ERR_INVALID_ARGUMENT, "the cache is NULL");
		if (buf < 0 || buf >= static_cast<int32_t>(kv->bufs.size()))
			return fail(NNC_ERR_INVALID_ARGUMENT, "buffer %d outside [0, %zu)", buf, kv->bufs.size());
		return NNC_OK;
	}

	nnc_status check_append(const nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, const void* k,
	                        const void* v)
	{
		if (nnc_status s = check_kv(kv, buf)) return s;
		if (!k || !v) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL K/V rows");
		if (n_tok <= 0 || pos0 < 0) return fail(NNC_ERR_INVALID_ARGUMENT, "append of %d rows at position %d", n_tok, pos0);
		if (n_tok > kv->bufs[buf].rows)
			return fail(NNC_ERR_INVALID_ARGUMENT, "%d rows do not fit a buffer of %d rows", n_tok, kv->bufs[buf].rows);
		return NNC_OK;
	}

	// Raw rows already in the element type: copy in at most two pieces
	// (before and after the ring's wrap).
	nnc_status append_raw(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, const void* k_rows,
	                      const void* v_rows, hipMemcpyKind kind)
	{
		const kv_buffer& b = kv->bufs[buf];
		const size_t row_bytes = static_cast<size_t>(b.kv_dim) * (kv->bf16 ? 2 : 4);
		int32_t done = 0;
		while (done < n_tok)
		{
			const int32_t row = (pos0 + done) % b.rows;
			const int32_t n = std::min(n_tok - done, b.rows - row);
			const size_t off = static_cast<size_t>(row) * row_bytes, src = static_cast<size_t>(done) * row_bytes;
			NNC_HIP_TRY(hipMemcpyAsync(static_cast<char*>(b.k) + off, static_cast<const char*>(k_rows) + src,
			                           n * row_bytes, kind, kv->stream),
			            "K/V append");
			NNC_HIP_TRY(hipMemcpyAsync(static_cast<char*>(b.v) + off, static_cast<const char*>(v_rows) + src,
			                           n * row_bytes, kind, kv->stream),
			            "K/V append");
			done += n;
		}
		if (b.v16)
		{
			nnchip::launch_shadow_rows(b.v, b.v16, kv->n_bad + buf, b.rows, b.kv_dim, pos0, n_tok,
			                           kv->stream);
			NNC_HIP_TRY(hipGetLastError(), "K/V append");
		}
		return NNC_OK;
	}

	// Shortest split, in wavefront chunks: what one CU keeps in flight
	// bounds a work-group's loads (about 17 bytes per clock measured with
	// 128 KiB per CU), so a short span goes to more work-groups with fewer
	// keys each rather than to fewer CUs.
	constexpr int kSplitFloorChunks = 1;
	// Most splits of one (token, head group): more work-groups than this
	// cost more in the merge than they gain (a one-KV-head layer at 8192
	// keys: 12.5 us with 128 splits, 15.5 with 256).
	constexpr long long kSplitsPerGroupMax = 128;

	// Keys per decode work-group for the span [kmin, kmax] shared out over
	// `pairs` (token, head group) pairs: about one work-group per CU (at
	// most kSplitsPerGroupMax per pair), a multiple of what one work-group
	// iteration consumes (wgk) or, for short spans, of one wavefront chunk
	// (unit), at most kDecodeMaxSplits splits.
	int split_keys_for(const nnc_hip_kv* kv, int kmin, int kmax, long long pairs, int wgk, int unit)
	{
		const int span = std::max(1, kmax - kmin + 1);
		const long long want =
			std::min(kSplitsPerGroupMax, std::max<long long>(1, 1LL * kv->n_cu / std::max<long long>(pairs, 1)));
		long long sk = (span + want - 1) / want;
		if (sk < wgk)
			sk = std::min<long long>(wgk, std::max<long long>(kSplitFloorChunks * unit, (sk + unit - 1) / unit * unit));
		else
			sk = (sk + wgk - 1) / wgk * wgk;
		while ((kmax / sk) - (kmin / sk) + 1 > nnchip::kDecodeMaxSplits) sk += sk < wgk ? unit : wgk;
		return static_cast<int>(sk);
	}

	// One split-K launch: tokens t0 .. t0 + n - 1 of a call on the absolute
	// split grid of sk keys.
	struct decode_plan
	{
		int32_t t0, n;
		int sk;
		bool tiled = false; // the tiled fp32-MFMA kernel instead of the per-token split-K kernels
		int nz = 0; // tiled: splits of the row block with the most keys (sk keys each, from the block's first key)
	};

	// Bytes of the tiled kernel's partials for a plan entry (none for one split).
	size_t tiled_part_bytes(const decode_plan& d, int32_t n_head, int32_t n_kv, int32_t head_dim)
	{
		if (d.nz <= 1) return 0;
		return static_cast<size_t>(d.n) * n_kv * d.nz * (n_head / n_kv) * (head_dim + 4) * sizeof(float);
	}

	// The split grid of one launch over tokens pos0 .. pos0 + n_tok - 1:
	// the first split's first key, the number of splits and the bytes of
	// partials it writes (none for one split); n_split 0 when no token sees a
	// key.
	struct launch_geometry
	{
		int split_base = 0, n_split = 0;
		size_t part_bytes = 0;
	};

	launch_geometry geometry_of(int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head,
	                            int32_t n_kv, int32_t head_dim, int split_keys)
	{
		launch_geometry g;
		int kmin, kmax, unused;
		nnchip::attn_span(causal ? 1 : 0, window, pos0, n_seq, kmin, unused);
		nnchip::attn_span(causal ? 1 : 0, window, pos0 + n_tok - 1, n_seq, unused, kmax);
		if (kmax < kmin) return g;
		g.split_base = (kmin / split_keys) * split_keys;
		g.n_split = kmax / split_keys - kmin / split_keys + 1;
		if (g.n_split > 1)
			g.part_bytes = static_cast<size_t>(n_tok) * n_kv * g.n_split * (n_head / n_kv) * (head_dim + 4) * sizeof(float);
		return g;
	}

	// One split-K launch (and its merge) over tokens pos0 .. pos0 + n_tok - 1
	// on the absolute split grid of split_keys keys. The partials go to
	// src (already checked to hold them) or to the cache's scratch.
	// One launch of the tiled kernel (plan entry d: its tokens, split size
	// and split count), partials in src or the cache's scratch.
	nnc_status tiled_launch(nnc_hip_kv* kv, const kv_buffer& b, const float* q, float* out, const float* gate,
	                        const decode_plan& d, int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head,
	                        int32_t n_kv, int32_t head_dim, float scale, const part_source& src)
	{
		const size_t bytes = tiled_part_bytes(d, n_head, n_kv, head_dim);
		float* part = src.ptr;
		if (!part && bytes)
		{
			if (nnc_status s = reserve(kv, kv->part, bytes, "tiled scratch")) return s;
			part = static_cast<float*>(kv->part.ptr);
		}
		nnchip::decode_params p{};
		p.q = q;
		p.out = out;
		p.gate = gate;
		p.K = b.k;
		p.V = b.v;
		p.part = part;
		p.rows = b.rows;
		p.kv_dim = b.kv_dim;
		p.n_head = n_head;
		p.n_kv = n_kv;
		p.pos0 = pos0;
		p.n_seq = n_seq;
		p.window = window;
		p.causal = causal ? 1 : 0;
		p.n_tok = d.n;
		p.split_keys = d.sk;
		p.n_split = d.nz;
		p.qscale = scale * 1.4426950408889634f;
		if (!nnchip::launch_tiled(p, d.n, head_dim, n_head / n_kv, kv->bf16, kv->stream))
			return fail(NNC_ERR_UNSUPPORTED_MODEL, "no tiled kernel for head_dim %d, group %d", head_dim, n_head / n_kv);
		NNC_HIP_TRY(hipGetLastError(), "tiled launch");
		return NNC_OK;
	}

	nnc_status decode_launch(nnc_hip_kv* kv, const kv_buffer& b, const float* q, float* out, const float* gate, int32_t n_tok,
	                         int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head, int32_t n_kv,
	                         int32_t head_dim, float scale, int split_keys, const part_source& src)
	{
		const int group = n_head / n_kv;
		const launch_geometry g = geometry_of(n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim, split_keys);
		if (g.n_split == 0)
			return nnchip::launch_zero(out, static_cast<size_t>(n_tok) * n_head * head_dim, kv->stream) ? NNC_OK
			                                                                                             : NNC_ERR_IO;
		if (g.n_split > nnchip::kDecodeMaxSplits)
			return fail(NNC_ERR_IO, "decode split grid of %d splits (at most %d)", g.n_split, nnchip::kDecodeMaxSplits);
		float* part = src.ptr;
		if (!part)
		{
			if (nnc_status s = reserve(kv, kv->part, g.part_bytes, "decode scratch")) return s;
			part = static_cast<float*>(kv->part.ptr);
		}

		nnchip::decode_params p{};
		p.q = q;
		p.out = out;
		p.gate = gate;
		p.K = b.k;
		p.V = b.v;
		p.part = part;
		p.rows = b.rows;
		p.kv_dim = b.kv_dim;
		p.n_head = n_head;
		p.n_kv = n_kv;
		p.pos0 = pos0;
		p.n_seq = n_seq;
		p.window = window;
		p.causal = causal ? 1 : 0;
		p.n_tok = n_tok;
		p.split_base = g.split_base;
		p.split_keys = split_keys;
		p.n_split = g.n_split;
		p.qscale = scale * 1.4426950408889634f;
		// One-token launches of the MFMA kernels over a few splits merge in
		// the split launch; the counts are the cache's, used in stream order.
		if (nnchip::mfma_shape(head_dim, group) && n_kv <= nnchip::kFuseCounts) p.counts = kv->counts;
		if (!nnchip::launch_decode(p, n_tok, head_dim, group, kv->bf16, kv->stream))
			return fail(NNC_ERR_UNSUPPORTED_MODEL, "no decode kernel for head_dim %d, group %d", head_dim, group);
		NNC_HIP_TRY(hipGetLastError(), "decode launch");
		return NNC_OK;
	}

	// The launches of a session-sized batch: each token on the split grid a
	// one-token call gives it (the split size of its own span over the head
	// groups). Consecutive tokens with the same split size share a launch; a
	// token's result does not depend on the rest of its launch, so it
	// matches the one-token call bit for bit.
	void plan_tokens(const nnc_hip_kv* kv, int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal,
	                 int32_t n_kv, int32_t head_dim, int group, std::vector<decode_plan>& plan)
	{
		const int wgk = nnchip::decode_wg_keys(head_dim, group, kv->bf16, n_kv);
		const int unit = nnchip::decode_chunk_keys(head_dim, group, kv->bf16);
		const int groups = nnchip::decode_groups(n_kv, kv->bf16, head_dim, group);
		auto span_of = [&](int32_t t, int& first, int& last)
		{ nnchip::attn_span(causal ? 1 : 0, window, pos0 + t, n_seq, first, last); };
		auto own_split = [&](int32_t t)
		{
			int first, last;
			span_of(t, first, last);
			return split_keys_for(kv, first, last, groups, wgk, unit);
		};
		for (int32_t t = 0; t < n_tok;)
		{
			const int sk = own_split(t);
			int f0, l0;
			span_of(t, f0, l0);
			int32_t u = t + 1;
			for (; u < n_tok && u - t < kDecodeChunk && own_split(u) == sk; ++u)
			{
				int fu, lu;
				span_of(u, fu, lu);
				if (lu / sk - f0 / sk + 1 > nnchip::kDecodeMaxSplits) break; // the launch's split grid stays mergeable
			}
			plan.push_back({t, u - t, sk});
			t = u;
		}
	}

	// The launches of an F32 batch of more than a session's tokens: chunks of
	// at most kDecodeChunk tokens (a grid z-extent and a scratch size that
	// stay small), each on the split grid of its own span.
	void plan_f32_chunks(const nnc_hip_kv* kv, int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal,
	                     int32_t n_kv, int32_t head_dim, int group, std::vector<decode_plan>& plan)
	{
		for (int32_t t0 = 0; t0 < n_tok; t0 += kDecodeChunk)
		{
			const int32_t nt = std::min(kDecodeChunk, n_tok - t0);
			int kmin, kmax, unused;
			nnchip::attn_span(causal ? 1 : 0, window, pos0 + t0, n_seq, kmin, unused);
			nnchip::attn_span(causal ? 1 : 0, window, pos0 + t0 + nt - 1, n_seq, unused, kmax);
			const int sk =
				split_keys_for(kv, kmin, kmax, static_cast<long long>(nt) * nnchip::decode_groups(n_kv, kv->bf16, head_dim, group),
				               nnchip::decode_wg_keys(head_dim, group, kv->bf16, n_kv),
				               nnchip::decode_chunk_keys(head_dim, group, kv->bf16));
			plan.push_back({t0, nt, sk});
		}
	}

	// The tiled kernel's launches: chunks of at most kTiledChunk tokens. Each
	// row block of 64 (token, head) rows splits its keys (the union of its
	// rows' spans) into splits of sk keys from its first key; sk is chosen so
	// that the work-groups of the launch about fill the part once (the
	// kernel's resident work-groups per CU: 4 up to head_dim 128, 2 up to
	// 256, else 1), at least 64 keys per split.
	void plan_tiled(const nnc_hip_kv* kv, int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal,
	                int32_t n_kv, int32_t head_dim, int group, std::vector<decode_plan>& plan)
	{
		const int per_cu = head_dim <= 128 ? 4 : head_dim <= 256 ? 2 : 1;
		for (int32_t t0 = 0; t0 < n_tok; t0 += kTiledChunk)
		{
			const int32_t nt = std::min(kTiledChunk, n_tok - t0);
			const long long n_rows = static_cast<long long>(nt) * group, n_blk = (n_rows + 63) / 64;
			std::vector<int> spans(static_cast<size_t>(n_blk));
			int max_span = 1;
			for (long long blk = 0; blk < n_blk; ++blk)
			{
				const long long r0 = 64 * blk, r1 = std::min(r0 + 64, n_rows) - 1;
				int lo, hi, unused;
				nnchip::attn_span(causal ? 1 : 0, window, pos0 + t0 + static_cast<int32_t>(r0 / group), n_seq, lo, unused);
				nnchip::attn_span(causal ? 1 : 0, window, pos0 + t0 + static_cast<int32_t>(r1 / group), n_seq, unused, hi);
				spans[static_cast<size_t>(blk)] = std::max(0, hi - lo + 1);
				max_span = std::max(max_span, hi - lo + 1);
			}
			const long long want = std::max<long long>(1, 1LL * kv->n_cu * per_cu / (n_blk * n_kv));
			long long sk = (max_span + want - 1) / want;
			sk = std::max<long long>(64, (sk + 15) / 16 * 16);
			int nz = 1;
			for (int sp : spans)
				if (sp > 0) nz = std::max(nz, static_cast<int>((sp - 1) / sk + 1));
			decode_plan d{t0, nt, static_cast<int>(sk), true, nz};
			plan.push_back(d);
		}
	}

	nnc_status attend_impl(nnc_hip_kv* kv, int32_t buf, const float* q, float* out, const float* gate, int32_t n_tok, int32_t pos0,
	                       int32_t n_seq, int32_t window, bool causal, int32_t n_head, int32_t n_kv, int32_t head_dim,
	                       float scale, const part_source& src = part_source{})
	{
		const kv_buffer& b = kv->bufs[buf];
		const int group = n_head / n_kv;
		const bool bf16 = kv->bf16;
		const size_t q_floats = static_cast<size_t>(n_tok) * n_head * head_dim;

		int first0, last0, first1, last1;
		nnchip::attn_span(causal ? 1 : 0, window, pos0, n_seq, first0, last0);
		nnchip::attn_span(causal ? 1 : 0, window, pos0 + n_tok - 1, n_seq, first1, last1);
		(void)last0;
		(void)first1;
		const int kmin = first0, kmax = last1;
		if (kmax < kmin) return nnchip::launch_zero(out, q_floats, kv->stream) ? NNC_OK : NNC_ERR_IO;

		// Decode and session-sized batches (and every batch in exact mode):
		// the split-K kernels, each token on its own split grid. Larger
		// batches: the MFMA prefill kernel for BF16 K/V of its head shapes;
		// the tiled fp32-MFMA kernel for F32 K/V and the other head shapes
		// with head_dim a multiple of 16 (exact fp32 products); otherwise the
		// split-K kernels (BF16: each token on its own grid; F32: over each
		// chunk's span).
		std::vector<decode_plan> plan;
		const bool mfma = nnchip::mfma_shape(head_dim, group), tiled = nnchip::tiled_shape_ok(head_dim, group);
		if (n_tok <= kSessionBatch || kv->exact_batches || (bf16 && !mfma && !tiled))
			plan_tokens(kv, n_tok, pos0, n_seq, window, causal, n_kv, head_dim, group, plan);
		else if (bf16 && mfma)
		{
			nnchip::prefill_params p{};
			p.q = q;
			p.out = out;
			p.gate = gate;
			p.K = b.k;
			p.V = b.v;
			p.V16 = b.v16;
			p.n_bad = b.v16 ? kv->n_bad + buf : nullptr;
			p.rows = b.rows;
			p.kv_dim = b.kv_dim;
			p.n_head = n_head;
			p.n_kv = n_kv;
			p.n_tok = n_tok;
			p.pos0 = pos0;
			p.n_seq = n_seq;
			p.window = window;
			p.causal = causal ? 1 : 0;
			p.qscale = scale * 1.4426950408889634f;
			if (!nnchip::launch_prefill(p, head_dim, group, bf16, kv->stream))
				return fail(NNC_ERR_UNSUPPORTED_MODEL, "no prefill kernel for head_dim %d, group %d", head_dim, group);
			NNC_HIP_TRY(hipGetLastError(), "prefill launch");
			return NNC_OK;
		}
		else if (tiled)
			plan_tiled(kv, n_tok, pos0, n_seq, window, causal, n_kv, head_dim, group, plan);
		else
			plan_f32_chunks(kv, n_tok, pos0, n_seq, window, causal, n_kv, head_dim, group, plan);

		// Every launch is planned before the first is enqueued: a call whose
		// partials do not fit the fixed scratch is refused whole.
		if (src.ptr)
			for (const decode_plan& d : plan)
			{
				const launch_geometry g =
					d.tiled ? launch_geometry{0, d.nz, tiled_part_bytes(d, n_head, n_kv, head_dim)}
					        : geometry_of(d.n, pos0 + d.t0, n_seq, window, causal, n_head, n_kv, head_dim, d.sk);
				if (g.part_bytes > src.bytes)
					return fail(NNC_ERR_INVALID_ARGUMENT,
					            "%d tokens over %d splits need %zu bytes of decode partials; the fixed scratch holds %zu",
					            d.n, g.n_split, g.part_bytes, src.bytes);
			}
		const size_t tok_floats = static_cast<size_t>(n_head) * head_dim;
		for (const decode_plan& d : plan)
		{
			const size_t off = static_cast<size_t>(d.t0) * tok_floats;
			nnc_status s = d.tiled ? tiled_launch(kv, b, q + off, out + off, gate ? gate + off : nullptr, d, pos0 + d.t0,
			                                      n_seq, window, causal, n_head, n_kv, head_dim, scale, src)
			                       : decode_launch(kv, b, q + off, out + off, gate ? gate + off : nullptr, d.n, pos0 + d.t0,
			                                       n_seq, window, causal, n_head, n_kv, head_dim, scale, d.sk, src);
			if (s) return s;
		}
		return NNC_OK;
	}

	nnc_status check_attend(const nnc_hip_kv* kv, int32_t buf, const float* q, const float* out, int32_t n_tok,
	                        int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head, int32_t n_kv,
	                        int32_t head_dim)
	{
		if (nnc_status s = check_kv(kv, buf)) return s;
		if (!q || !out) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL q or out");
		if (n_tok <= 0 || pos0 < 0 || n_seq < 1 || window < 0)
			return fail(NNC_ERR_INVALID_ARGUMENT, "bad batch: %d tokens at %d, n_seq %d, window %d", n_tok, pos0, n_seq,
			            window);
		if (n_kv <= 0 || n_head <= 0 || n_head % n_kv != 0 || head_dim <= 0)
			return fail(NNC_ERR_INVALID_ARGUMENT, "bad heads: %d query heads over %d KV heads, head_dim %d", n_head,
			            n_kv, head_dim);
		const kv_buffer& b = kv->bufs[buf];
		if (static_cast<long long>(n_kv) * head_dim != b.kv_dim)
			return fail(NNC_ERR_INVALID_ARGUMENT, "%d KV heads of %d do not make the buffer's kv_dim %d", n_kv, head_dim,
			            b.kv_dim);
		const int group = n_head / n_kv;
		if (!nnchip::mfma_shape(head_dim, group) && !nnchip::generic_shape_ok(head_dim, group))
			return fail(NNC_ERR_UNSUPPORTED_MODEL,
			            "head_dim %d with group %d is not supported on the GPU (an even head_dim up to 512, group up to "
			            "%d, group * head_dim up to %d)",
			            head_dim, group, nnchip::kGenMaxGroup, nnchip::kGenMaxGroupDim);
		if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out)) & 15)
			return fail(NNC_ERR_INVALID_ARGUMENT, "q and out must be 16-byte aligned");
		// The BF16 kernels address a buffer with 32-bit byte offsets.
		if (kv->bf16 && static_cast<uint64_t>(b.rows) * b.kv_dim * 2 > 0x7fffffffu)
			return fail(NNC_ERR_UNSUPPORTED_MODEL, "a %d x %d BF16 buffer is too large for the GPU kernels (2 GiB)",
			            b.rows, b.kv_dim);
		// Every key the batch reads must still be in the buffer: the newest
		// position written is n_seq - 1, and the buffer keeps the last `rows`.
		int first0, last0;
		nnchip::attn_span(causal ? 1 : 0, window, pos0, n_seq, first0, last0);
		(void)last0;
		if (static_cast<long long>(n_seq) - first0 > b.rows)
			return fail(NNC_ERR_CONTEXT_FULL, "keys %d .. %d do not fit a buffer of %d rows", first0, n_seq - 1, b.rows);
		return NNC_OK;
	}
	// The device address of `scratch` on `device`: looked up once per device,
	// with that device current, when the first cache on it is created (the
	// library's set-up; a later no-alloc call only reads the table).
	nnc_status noalloc_scratch(int device, void** out)
	{
		if (device < 0 || device >= kMaxDevices)
			return fail(NNC_ERR_UNSUPPORTED_CPU, "device %d is past the library's %d-device table", device, kMaxDevices);
		std::lock_guard<std::mutex> lock(g_scratch_mu);
		if (!g_scratch_ptr[device])
		{
			int cur = 0;
			NNC_HIP_TRY(hipGetDevice(&cur), "scratch lookup");
			if (cur != device) NNC_HIP_TRY(hipSetDevice(device), "scratch lookup");
			void* ptr = nullptr;
			const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
			if (cur != device) (void)hipSetDevice(cur);
			if (e != hipSuccess) return hip_fail(e, "scratch lookup");
			if (!ptr) return fail(NNC_ERR_IO, "scratch lookup: no device address");
			g_scratch_ptr[device] = ptr;
		}
		*out = g_scratch_ptr[device];
		return NNC_OK;
	}
}

extern "C" {

nnc_status nnc_hip_kv_create(int32_t n_buf, const int32_t* rows, const int32_t* kv_dim, bool bf16, nnc_hip_kv** out)
{
	if (!out) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL output handle");
	*out = nullptr;
	if (n_buf <= 0 || !rows || !kv_dim) return fail(NNC_ERR_INVALID_ARGUMENT, "%d buffers, rows or kv_dim NULL", n_buf);
	for (int32_t i = 0; i < n_buf; ++i)
		if (rows[i] <= 0 || kv_dim[i] <= 0 || kv_dim[i] % 8 != 0)
			return fail(NNC_ERR_INVALID_ARGUMENT, "buffer %d: %d rows of %d elements (kv_dim must be a positive multiple of 8)",
			            i, rows[i], kv_dim[i]);
	int n_dev = 0;
	if (hipGetDeviceCount(&n_dev) != hipSuccess || n_dev <= 0)
		return fail(NNC_ERR_UNSUPPORTED_CPU, "no HIP device is available");

	nnc_hip_kv* kv = new (std::nothrow) nnc_hip_kv();
	if (!kv) return fail(NNC_ERR_OUT_OF_MEMORY, "out of host memory");
	kv->bf16 = bf16;
	auto bail = [&](nnc_status s)
	{
		release(kv);
		return s;
	};
	hipError_t e = hipGetDevice(&kv->device);
	if (e == hipSuccess) e = hipDeviceGetAttribute(&kv->n_cu, hipDeviceAttributeMultiprocessorCount, kv->device);
	if (e == hipSuccess) e = hipStreamCreateWithFlags(&kv->stream, hipStreamNonBlocking);
	if (e == hipSuccess) e = hipEventCreateWithFlags(&kv->pinned.free, hipEventDisableTiming);
	if (e != hipSuccess) return bail(hip_fail(e, "device setup"));
	const size_t esize = bf16 ? 2 : 4;
	const bool shadow = bf16 && f16_shadow_enabled();
	kv->bufs.resize(static_cast<size_t>(n_buf));
	if (shadow)
	{
		e = hipMalloc(&kv->n_bad, sizeof(int) * static_cast<size_t>(n_buf));
		if (e == hipSuccess) e = hipMemsetAsync(kv->n_bad, 0, sizeof(int) * static_cast<size_t>(n_buf), kv->stream);
		if (e != hipSuccess) return bail(hip_fail(e, "K/V allocation"));
	}
	for (int32_t i = 0; i < n_buf; ++i)
	{
		kv_buffer& b = kv->bufs[i];
		b.rows = rows[i];
		b.kv_dim = kv_dim[i];
		const size_t n = static_cast<size_t>(rows[i]) * kv_dim[i] * esize;
		e = hipMalloc(&b.k, n);
		if (e == hipSuccess) e = hipMalloc(&b.v_alloc, n + kVOffset);
		if (e == hipSuccess) b.v = static_cast<char*>(b.v_alloc) + kVOffset;
		if (e == hipSuccess) e = hipMemsetAsync(b.k, 0, n, kv->stream);
		if (e == hipSuccess) e = hipMemsetAsync(b.v, 0, n, kv->stream);
		if (shadow)
		{
			// zeroed: rows never written hold finite values, which the prefill
			// kernels may read (and weigh 0) beside a group's written rows
			const size_t n16 = nnchip::f16_copy_bytes(rows[i], kv_dim[i]);
			if (e == hipSuccess) e = hipMalloc(&b.v16_alloc, n16 + kVOffset);
			if (e == hipSuccess) b.v16 = static_cast<char*>(b.v16_alloc) + kVOffset;
			if (e == hipSuccess) e = hipMemsetAsync(b.v16, 0, n16, kv->stream);
			kv->bytes += n16;
		}
		if (e != hipSuccess) return bail(hip_fail(e, "K/V allocation"));
		kv->bytes += 2 * n;
	}
	e = hipMalloc(&kv->counts, sizeof(unsigned) * nnchip::kFuseCounts);
	if (e == hipSuccess) e = hipMemsetAsync(kv->counts, 0, sizeof(unsigned) * nnchip::kFuseCounts, kv->stream);
	if (e == hipSuccess) e = hipStreamSynchronize(kv->stream);
	if (e != hipSuccess) return bail(hip_fail(e, "K/V allocation"));
	void* fixed = nullptr;
	if (nnc_status s = noalloc_scratch(kv->device, &fixed)) return bail(s);
	// The counterpart of nnc's context line (reference session.cpp:341-343).
	hipDeviceProp_t prop;
	const bool named = hipGetDeviceProperties(&prop, kv->device) == hipSuccess;
	log_msg(NNC_HIP_LOG_INFO, "device %d (%s, %d CUs): %d K/V buffers, %.1f MB of %s K/V%s in device memory",
	        kv->device, named ? prop.name : "unknown", kv->n_cu, n_buf, static_cast<double>(kv->bytes) / 1e6,
	        bf16 ? "BF16" : "F32", shadow ? " (with V's fp16 copy)" : "");
	*out = kv;
	return NNC_OK;
}

void nnc_hip_kv_free(nnc_hip_kv* kv) { release(kv); }

void nnc_hip_set_log_callback(nnc_hip_log_callback callback, void* user)
{
	std::lock_guard<std::mutex> lock(g_log_mu);
	g_log_cb = callback;
	g_log_user = user;
}

uint64_t nnc_hip_kv_bytes(const nnc_hip_kv* kv) { return kv ? kv->bytes : 0; }

nnc_status nnc_hip_kv_set_exact_batches(nnc_hip_kv* kv, bool exact)
{
	if (!kv) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL cache");
	kv->exact_batches = exact;
	return NNC_OK;
}

nnc_status nnc_hip_kv_append(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, const void* k_rows,
                             const void* v_rows)
{
	if (nnc_status s = check_append(kv, buf, pos0, n_tok, k_rows, v_rows)) return s;
	// Through the pinned staging, straight into the buffer's rows, so the
	// host rows are free on return.
	const size_t bytes = static_cast<size_t>(n_tok) * kv->bufs[buf].kv_dim * (kv->bf16 ? 2 : 4);
	if (nnc_status s = reserve_pinned(kv, 2 * bytes, "append staging")) return s;
	char* pk = static_cast<char*>(kv->pinned.ptr);
	std::memcpy(pk, k_rows, bytes);
	std::memcpy(pk + bytes, v_rows, bytes);
	if (nnc_status s = append_raw(kv, buf, pos0, n_tok, pk, pk + bytes, hipMemcpyHostToDevice)) return s;
	NNC_HIP_TRY(hipEventRecord(kv->pinned.free, kv->stream), "K/V append");
	return NNC_OK;
}

nnc_status nnc_hip_kv_append_f32(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, const float* k_rows,
                                 const float* v_rows)
{
	if (nnc_status s = check_append(kv, buf, pos0, n_tok, k_rows, v_rows)) return s;
	const size_t bytes = static_cast<size_t>(n_tok) * kv->bufs[buf].kv_dim * sizeof(float);
	if (nnc_status s = reserve(kv, kv->rows_k, bytes, "append staging")) return s;
	if (nnc_status s = reserve(kv, kv->rows_v, bytes, "append staging")) return s;
	if (nnc_status s = reserve_pinned(kv, 2 * bytes, "append staging")) return s;
	char* pk = static_cast<char*>(kv->pinned.ptr);
	std::memcpy(pk, k_rows, bytes);
	std::memcpy(pk + bytes, v_rows, bytes);
	NNC_HIP_TRY(hipMemcpyAsync(kv->rows_k.ptr, pk, bytes, hipMemcpyHostToDevice, kv->stream), "K/V append");
	NNC_HIP_TRY(hipMemcpyAsync(kv->rows_v.ptr, pk + bytes, bytes, hipMemcpyHostToDevice, kv->stream), "K/V append");
	NNC_HIP_TRY(hipEventRecord(kv->pinned.free, kv->stream), "K/V append");
	return nnc_hip_kv_append_f32_device(kv, buf, pos0, n_tok, static_cast<const float*>(kv->rows_k.ptr),
	                                    static_cast<const float*>(kv->rows_v.ptr));
}

nnc_status nnc_hip_kv_append_f32_device(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, const float* k_rows,
                                        const float* v_rows)
{
	if (nnc_status s = check_append(kv, buf, pos0, n_tok, k_rows, v_rows)) return s;
	const kv_buffer& b = kv->bufs[buf];
	nnchip::launch_append_f32(b.k, b.v, k_rows, v_rows, b.rows, b.kv_dim, pos0, n_tok, kv->bf16, kv->stream, b.v16,
	                          b.v16 ? kv->n_bad + buf : nullptr);
	NNC_HIP_TRY(hipGetLastError(), "K/V append");
	return NNC_OK;
}

nnc_status nnc_hip_kv_prep_append_device(nnc_hip_kv* kv, int32_t buf, int32_t pos0, int32_t n_tok, float* q,
                                         const float* k, const float* v, const nnc_hip_prep* prep)
{
	if (nnc_status s = check_kv(kv, buf)) return s;
	if (!q || !k || !v || !prep) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL q, k, v or parameters");
	const kv_buffer& b = kv->bufs[buf];
	if (n_tok <= 0 || pos0 < 0) return fail(NNC_ERR_INVALID_ARGUMENT, "n_tok %d, pos0 %d", n_tok, pos0);
	if (n_tok > b.rows)
		return fail(NNC_ERR_INVALID_ARGUMENT, "%d tokens overwrite each other in a buffer of %d rows", n_tok, b.rows);
	const nnc_hip_prep& pr = *prep;
	if (pr.n_head <= 0 || pr.n_kv <= 0 || pr.head_dim <= 0)
		return fail(NNC_ERR_INVALID_ARGUMENT, "n_head %d, n_kv %d, head_dim %d", pr.n_head, pr.n_kv, pr.head_dim);
	if (static_cast<long long>(pr.n_kv) * pr.head_dim != b.kv_dim)
		return fail(NNC_ERR_INVALID_ARGUMENT, "n_kv * head_dim = %lld, buffer kv_dim %d",
		            static_cast<long long>(pr.n_kv) * pr.head_dim, b.kv_dim);
	if (pr.n_rot < 0 || pr.n_rot % 2 != 0 || pr.n_rot > pr.head_dim)
		return fail(NNC_ERR_INVALID_ARGUMENT, "n_rot %d (even, at most head_dim %d)", pr.n_rot, pr.head_dim);
	if (pr.rope_mode != 0 && pr.rope_mode != 1) return fail(NNC_ERR_INVALID_ARGUMENT, "rope_mode %d", pr.rope_mode);
	if (pr.n_rot > 0 && !(pr.freq_base > 0.0f)) return fail(NNC_ERR_INVALID_ARGUMENT, "freq_base %g", pr.freq_base);
	if (pr.head_dim > 2 * nnchip::kPrepMaxPairs)
		return fail(NNC_ERR_UNSUPPORTED_MODEL, "head_dim %d above %d", pr.head_dim, 2 * nnchip::kPrepMaxPairs);

	nnchip::prep_params p{};
	p.q = q;
	p.k = k;
	p.v = v;
	p.K = b.k;
	p.V = b.v;
	p.V16 = b.v16;
	p.n_bad = b.v16 ? kv->n_bad + buf : nullptr;
	p.q_gamma = pr.q_gamma;
	p.k_gamma = pr.k_gamma;
	p.n_head = pr.n_head;
	p.n_kv = pr.n_kv;
	p.head_dim = pr.head_dim;
	p.rows = b.rows;
	p.pos0 = pos0;
	p.bf16 = kv->bf16 ? 1 : 0;
	p.v_norm = pr.v_norm ? 1 : 0;
	p.n_rot = pr.n_rot;
	p.mode = pr.rope_mode;
	p.eps = pr.rms_eps;
	p.inv_dim = 1.0f / static_cast<float>(pr.head_dim); // (reference nn_ops.cpp:594)
	p.rope_cs = nullptr;
	if (pr.n_rot > 0)
		if (nnc_status s = rope_cs(kv, pr, pos0, n_tok, p.rope_cs)) return s;
	if (!nnchip::launch_prep(p, n_tok, kv->stream))
		return fail(NNC_ERR_UNSUPPORTED_MODEL, "no pre-attention kernel for head_dim %d", pr.head_dim);
	NNC_HIP_TRY(hipGetLastError(), "pre-attention step");
	return NNC_OK;
}

nnc_status nnc_hip_kv_read(nnc_hip_kv* kv, int32_t buf, int32_t row0, int32_t n_rows, void* k_out, void* v_out)
{
	if (nnc_status s = check_kv(kv, buf)) return s;
	const kv_buffer& b = kv->bufs[buf];
	if (row0 < 0 || n_rows < 0 || row0 + static_cast<long long>(n_rows) > b.rows)
		return fail(NNC_ERR_INVALID_ARGUMENT, "rows %d .. %d outside a buffer of %d", row0, row0 + n_rows - 1, b.rows);
	const size_t row_bytes = static_cast<size_t>(b.kv_dim) * (kv->bf16 ? 2 : 4);
	const size_t off = static_cast<size_t>(row0) * row_bytes, n = static_cast<size_t>(n_rows) * row_bytes;
	if (k_out && n)
		NNC_HIP_TRY(hipMemcpyAsync(k_out, static_cast<char*>(b.k) + off, n, hipMemcpyDeviceToHost, kv->stream), "K/V read");
	if (v_out && n)
		NNC_HIP_TRY(hipMemcpyAsync(v_out, static_cast<char*>(b.v) + off, n, hipMemcpyDeviceToHost, kv->stream), "K/V read");
	NNC_HIP_TRY(hipStreamSynchronize(kv->stream), "K/V read");
	return NNC_OK;
}

namespace
{
	// The host-buffer form of the op: q (and gate) staged to the device
	// through pinned memory, out downloaded through it, the call synchronous
	// with respect to out.
	static nnc_status attend_host(nnc_hip_kv* kv, int32_t buf, const float* q, const float* gate, float* out, int32_t n_tok,
	                       int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head, int32_t n_kv,
	                       int32_t head_dim, float scale)
	{
		// Host pointers need no alignment: they are staged.
		static const float aligned_probe[4] = {0, 0, 0, 0};
		if (nnc_status s = check_attend(kv, buf, q ? aligned_probe : nullptr, out ? aligned_probe : nullptr, n_tok,
		                                pos0, n_seq, window, causal, n_head, n_kv, head_dim))
			return s;
		const size_t n = static_cast<size_t>(n_tok) * n_head * head_dim, bytes = n * sizeof(float);
		const size_t slot = (bytes + 255) & ~static_cast<size_t>(255);
		if (nnc_status s = reserve(kv, kv->q, bytes, "q staging")) return s;
		if (gate)
			if (nnc_status s = reserve(kv, kv->gate, bytes, "gate staging")) return s;
		// pinned: q, gate, then out (written by the kernels themselves)
		if (nnc_status s = reserve_pinned(kv, 3 * slot, "q staging")) return s;
		char* pq = static_cast<char*>(kv->pinned.ptr);
		float* pout = reinterpret_cast<float*>(pq + 2 * slot);
		std::memcpy(pq, q, bytes);
		nnchip::launch_copy(static_cast<float*>(kv->q.ptr), reinterpret_cast<const float*>(pq), n, kv->stream);
		if (gate)
		{
			std::memcpy(pq + slot, gate, bytes);
			nnchip::launch_copy(static_cast<float*>(kv->gate.ptr), reinterpret_cast<const float*>(pq + slot), n,
			                    kv->stream);
		}
		NNC_HIP_TRY(hipGetLastError(), "q upload");
		if (nnc_status s = attend_impl(kv, buf, static_cast<const float*>(kv->q.ptr), pout,
		                               gate ? static_cast<const float*>(kv->gate.ptr) : nullptr, n_tok, pos0, n_seq,
		                               window, causal, n_head, n_kv, head_dim, scale))
		{
			(void)hipStreamSynchronize(kv->stream); // the staging is read until the uploads finish
			return s;
		}
		NNC_HIP_TRY(hipStreamSynchronize(kv->stream), "attention");
		std::memcpy(out, pout, bytes);
		return NNC_OK;
	}
}

nnc_status nnc_hip_attend(nnc_hip_kv* kv, int32_t buf, const float* q, float* out, int32_t n_tok, int32_t pos0,
                          int32_t n_seq, int32_t window, bool causal, int32_t n_head, int32_t n_kv, int32_t head_dim,
                          float scale)
{
	return attend_host(kv, buf, q, nullptr, out, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim, scale);
}

nnc_status nnc_hip_attend_device(nnc_hip_kv* kv, int32_t buf, const float* q, float* out, int32_t n_tok, int32_t pos0,
                                 int32_t n_seq, int32_t window, bool causal, int32_t n_head, int32_t n_kv,
                                 int32_t head_dim, float scale)
{
	if (nnc_status s = check_attend(kv, buf, q, out, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim))
		return s;
	return attend_impl(kv, buf, q, out, nullptr, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim, scale);
}

nnc_status nnc_hip_attend_device_noalloc(nnc_hip_kv* kv, int32_t buf, const float* q, float* out, int32_t n_tok,
                                         int32_t pos0, int32_t n_seq, int32_t window, bool causal, int32_t n_head,
                                         int32_t n_kv, int32_t head_dim, float scale)
{
	if (nnc_status s = check_attend(kv, buf, q, out, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim))
		return s;
	void* ptr = nullptr;
	if (nnc_status s = noalloc_scratch(kv->device, &ptr)) return s;
	part_source src;
	src.ptr = static_cast<float*>(ptr);
	src.bytes = NNC_HIP_NOALLOC_SCRATCH_BYTES;
	return attend_impl(kv, buf, q, out, nullptr, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim, scale, src);
}

nnc_status nnc_hip_attend_gated(nnc_hip_kv* kv, int32_t buf, const float* q, const float* gate, float* out,
                                int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal,
                                int32_t n_head, int32_t n_kv, int32_t head_dim, float scale)
{
	if (!gate) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL gate");
	return attend_host(kv, buf, q, gate, out, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim, scale);
}

nnc_status nnc_hip_attend_gated_device(nnc_hip_kv* kv, int32_t buf, const float* q, const float* gate, float* out,
                                       int32_t n_tok, int32_t pos0, int32_t n_seq, int32_t window, bool causal,
                                       int32_t n_head, int32_t n_kv, int32_t head_dim, float scale)
{
	if (!gate) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL gate");
	if (nnc_status s = check_attend(kv, buf, q, out, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim))
		return s;
	return attend_impl(kv, buf, q, out, gate, n_tok, pos0, n_seq, window, causal, n_head, n_kv, head_dim, scale);
}

namespace
{
	// p.mrow and p.rows for n matrices of the given row counts, stacked.
	static void stack_rows(nnchip::gemv_params& p, const uint32_t* rows, int n)
	{
		int acc = 0;
		p.mrow[0] = 0;
		for (int m = 0; m < n; ++m)
		{
			acc += static_cast<int>(rows[m]);
			p.mrow[m + 1] = acc;
		}
		for (int m = n + 1; m <= nnchip::kGemvMaxMats; ++m) p.mrow[m] = INT_MAX;
		p.rows = acc;
	}

	// Weight gemvs over the same X on the context's stream: one launch per
	// chunk of at most kGemvMaxBatch vectors for all the matrices together
	// (stacked along the rows), or one per matrix when a matrix other than
	// the last has a row count that is not a multiple of 16.
	static nnc_status gemv_impl(nnc_hip_kv* kv, int format, int n_mat, const nnc_hip_gemv_mat* mats, const float* X,
	                     size_t x_stride, const float* XSUM, size_t xsum_stride, uint32_t cols, uint32_t n_batch)
	{
		if (!kv) return fail(NNC_ERR_INVALID_ARGUMENT, "the context (cache) is NULL");
		if (format != nnchip::kGemvBf16 && format != nnchip::kGemvQ8_0 && format != nnchip::kGemvQ4S)
			return fail(NNC_ERR_INVALID_ARGUMENT, "gemv format %d", format);
		if (!mats || n_mat < 1 || n_mat > nnchip::kGemvMaxMats)
			return fail(NNC_ERR_INVALID_ARGUMENT, "%d matrices in a gemv group (1 to %d)", n_mat, nnchip::kGemvMaxMats);
		if (!X) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL input pointer");
		uint64_t total = 0;
		bool stackable = true;
		for (int m = 0; m < n_mat; ++m)
		{
			const nnc_hip_gemv_mat& M = mats[m];
			if (!M.w || !M.y || (format != nnchip::kGemvBf16 && !M.scales) || (format == nnchip::kGemvQ4S && !M.biases))
				return fail(NNC_ERR_INVALID_ARGUMENT, "NULL weight, scale, bias or output pointer (matrix %d)", m);
			if (M.rows > 0x7fffffffu) return fail(NNC_ERR_INVALID_ARGUMENT, "gemv of %u rows", M.rows);
			if (M.y_stride < M.rows)
				return fail(NNC_ERR_INVALID_ARGUMENT, "y_stride %zu below %u rows (matrix %d)", M.y_stride, M.rows, m);
			if (reinterpret_cast<uintptr_t>(M.w) & 15)
				return fail(NNC_ERR_INVALID_ARGUMENT, "weights must be 16-byte aligned (matrix %d)", m);
			total += M.rows;
			if (m + 1 < n_mat && M.rows % 16 != 0) stackable = false;
		}
		if (total == 0 || cols == 0 || n_batch == 0) return NNC_OK; // nothing to do, as in the reference
		if (total > 0x7fffffffu || cols > 0x7fffffffu)
			return fail(NNC_ERR_INVALID_ARGUMENT, "gemv of %llu x %u", static_cast<unsigned long long>(total), cols);
		if (cols % 32 != 0)
			return fail(NNC_ERR_UNSUPPORTED_MODEL, "gemv with %u columns (a multiple of 32 is required)", cols);
		if (x_stride < cols || (format == nnchip::kGemvQ4S && XSUM && xsum_stride < cols / 32))
			return fail(NNC_ERR_INVALID_ARGUMENT, "strides %zu / %zu for %u columns", x_stride, xsum_stride, cols);
		if ((reinterpret_cast<uintptr_t>(X) & 15) || x_stride % 4 != 0)
			return fail(NNC_ERR_INVALID_ARGUMENT, "X must be 16-byte aligned, x_stride a multiple of 4");
		if (!stackable)
		{
			for (int m = 0; m < n_mat; ++m)
				if (nnc_status s = gemv_impl(kv, format, 1, mats + m, X, x_stride, XSUM, xsum_stride, cols, n_batch))
					return s;
			return NNC_OK;
		}
		uint32_t rows[nnchip::kGemvMaxMats];
		for (int m = 0; m < n_mat; ++m) rows[m] = mats[m].rows;
		for (uint32_t t0 = 0; t0 < n_batch; t0 += nnchip::kGemvMaxBatch)
		{
			const int nb = static_cast<int>(std::min<uint32_t>(n_batch - t0, nnchip::kGemvMaxBatch));
			nnchip::gemv_params p{};
			p.format = format;
			stack_rows(p, rows, n_mat);
			int n_split = 1, split_blocks = 1;
			nnchip::gemv_plan(p.rows, static_cast<int>(cols), nb, format, n_split, split_blocks);
			if (n_split > 1)
				if (nnc_status s = reserve(kv, kv->gemv_part,
				                           static_cast<size_t>(n_split) * nb * static_cast<size_t>(p.rows) * sizeof(float),
				                           "gemv scratch"))
					return s;
			for (int m = 0; m < n_mat; ++m)
			{
				const nnc_hip_gemv_mat& M = mats[m];
				p.mats[m] = nnchip::gemv_mat{M.w, M.scales, M.biases, M.y + t0 * M.y_stride, M.y_stride};
			}
			p.x = X + t0 * x_stride;
			p.xsum = XSUM ? XSUM + t0 * xsum_stride : nullptr;
			p.part = static_cast<float*>(kv->gemv_part.ptr);
			p.x_stride = x_stride;
			p.xsum_stride = xsum_stride;
			p.cols = static_cast<int>(cols);
			p.n_batch = nb;
			p.n_split = n_split;
			p.split_blocks = split_blocks;
			if (!nnchip::launch_gemv(p, kv->stream)) return fail(NNC_ERR_UNSUPPORTED_MODEL, "gemv format %d", format);
			NNC_HIP_TRY(hipGetLastError(), "gemv launch");
		}
		return NNC_OK;
	}
}

nnc_status nnc_hip_gemv_bf16_argmax(nnc_hip_kv* kv, const void* W, const float* x, uint32_t rows, uint32_t cols,
                                    int32_t* index)
{
	if (!kv) return fail(NNC_ERR_INVALID_ARGUMENT, "the context (cache) is NULL");
	if (!W || !x || !index) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL weight, input or index pointer");
	if (rows == 0 || cols == 0)
	{
		*index = -1; // reference nn_ops.cpp:1058
		return NNC_OK;
	}
	if (rows > 0x7fffffffu || cols > 0x7fffffffu) return fail(NNC_ERR_INVALID_ARGUMENT, "gemv of %u x %u", rows, cols);
	if (cols % 32 != 0 || !nnchip::gemv_vec_fits(static_cast<int>(cols), 1, nnchip::kGemvBf16))
		return fail(NNC_ERR_UNSUPPORTED_MODEL, "argmax gemv with %u columns (a multiple of 32, at most 15872)", cols);
	if ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x)) & 15)
		return fail(NNC_ERR_INVALID_ARGUMENT, "weights and x must be 16-byte aligned");
	const int groups = nnchip::gemv_vec_groups(static_cast<int>(rows));
	const size_t best_bytes = static_cast<size_t>(groups) * sizeof(float2);
	if (nnc_status s = reserve(kv, kv->gemv_part, best_bytes + 2 * sizeof(int32_t), "gemv scratch")) return s;
	nnchip::gemv_params p{};
	p.format = nnchip::kGemvBf16;
	p.first_sticks = rows % 4 != 0; // the reference's fallback scans from y[0] (nn_ops.cpp:1184-1196)
	p.mats[0].w = W;
	stack_rows(p, &rows, 1);
	p.x = x;
	p.x_stride = cols;
	p.cols = static_cast<int>(cols);
	p.n_batch = 1;
	p.n_split = 1;
	p.split_blocks = static_cast<int>(cols / 32);
	p.best = static_cast<float2*>(kv->gemv_part.ptr);
	p.argmax = reinterpret_cast<int*>(static_cast<char*>(kv->gemv_part.ptr) + best_bytes);
	if (!nnchip::launch_gemv_argmax(p, kv->stream)) return fail(NNC_ERR_UNSUPPORTED_MODEL, "argmax gemv");
	NNC_HIP_TRY(hipGetLastError(), "argmax gemv launch");
	int32_t r = 0;
	NNC_HIP_TRY(hipMemcpyAsync(&r, p.argmax, sizeof(r), hipMemcpyDeviceToHost, kv->stream), "argmax download");
	NNC_HIP_TRY(hipStreamSynchronize(kv->stream), "argmax gemv");
	*index = r;
	return NNC_OK;
}

nnc_status nnc_hip_argmax_f32(nnc_hip_kv* kv, const float* y, uint32_t n, int32_t* index)
{
	if (!kv) return fail(NNC_ERR_INVALID_ARGUMENT, "the context (cache) is NULL");
	if (!y || !index) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL input or index pointer");
	if (n == 0)
	{
		*index = 0; // the reference's scan starts at row 0 (model.cpp:2192-2194)
		return NNC_OK;
	}
	if (n > 0x7fffffffu) return fail(NNC_ERR_INVALID_ARGUMENT, "argmax of %u elements", n);
	const size_t best_bytes = static_cast<size_t>(nnchip::kArgmaxGroups) * sizeof(float2);
	if (nnc_status s = reserve(kv, kv->gemv_part, best_bytes + 2 * sizeof(int32_t), "gemv scratch")) return s;
	nnchip::gemv_params p{};
	p.mats[0].y = const_cast<float*>(y);
	stack_rows(p, &n, 1);
	p.best = static_cast<float2*>(kv->gemv_part.ptr);
	p.argmax = reinterpret_cast<int*>(static_cast<char*>(kv->gemv_part.ptr) + best_bytes);
	p.first_sticks = 1;
	nnchip::launch_argmax(p, kv->stream);
	NNC_HIP_TRY(hipGetLastError(), "argmax launch");
	int32_t r = 0;
	NNC_HIP_TRY(hipMemcpyAsync(&r, p.argmax, sizeof(r), hipMemcpyDeviceToHost, kv->stream), "argmax download");
	NNC_HIP_TRY(hipStreamSynchronize(kv->stream), "argmax");
	*index = r;
	return NNC_OK;
}

nnc_status nnc_hip_gemv_bf16(nnc_hip_kv* kv, const void* W, const float* X, size_t x_stride, float* Y, size_t y_stride,
                             uint32_t rows, uint32_t cols, uint32_t n_batch)
{
	const nnc_hip_gemv_mat m{W, nullptr, nullptr, Y, y_stride, rows};
	return gemv_impl(kv, nnchip::kGemvBf16, 1, &m, X, x_stride, nullptr, 0, cols, n_batch);
}

nnc_status nnc_hip_gemv_q8_0(nnc_hip_kv* kv, const int8_t* qs, const uint16_t* scales, const float* X,
                             size_t x_stride, float* Y, size_t y_stride, uint32_t rows, uint32_t cols,
                             uint32_t n_batch)
{
	const nnc_hip_gemv_mat m{qs, scales, nullptr, Y, y_stride, rows};
	return gemv_impl(kv, nnchip::kGemvQ8_0, 1, &m, X, x_stride, nullptr, 0, cols, n_batch);
}

nnc_status nnc_hip_gemv_q4_s(nnc_hip_kv* kv, const uint8_t* qs, const uint16_t* scales, const uint16_t* biases,
                             const float* X, size_t x_stride, const float* XSUM, size_t xsum_stride, float* Y,
                             size_t y_stride, uint32_t rows, uint32_t cols, uint32_t n_batch)
{
	const nnc_hip_gemv_mat m{qs, scales, biases, Y, y_stride, rows};
	return gemv_impl(kv, nnchip::kGemvQ4S, 1, &m, X, x_stride, XSUM, xsum_stride, cols, n_batch);
}

nnc_status nnc_hip_gemv_group(nnc_hip_kv* kv, int32_t format, int32_t n_mat, const nnc_hip_gemv_mat* mats,
                              const float* X, size_t x_stride, const float* XSUM, size_t xsum_stride, uint32_t cols,
                              uint32_t n_batch)
{
	static_assert(NNC_HIP_GEMV_BF16 == nnchip::kGemvBf16 && NNC_HIP_GEMV_Q8_0 == nnchip::kGemvQ8_0 &&
	                  NNC_HIP_GEMV_Q4_S == nnchip::kGemvQ4S && NNC_HIP_GEMV_MAX_GROUP == nnchip::kGemvMaxMats,
	              "format codes");
	return gemv_impl(kv, format, n_mat, mats, X, x_stride, format == nnchip::kGemvQ4S ? XSUM : nullptr, xsum_stride, cols,
	                 n_batch);
}

nnc_status nnc_hip_kv_sync(nnc_hip_kv* kv)
{
	if (!kv) return fail(NNC_ERR_INVALID_ARGUMENT, "the cache is NULL");
	NNC_HIP_TRY(hipStreamSynchronize(kv->stream), "stream sync");
	return NNC_OK;
}

void* nnc_hip_kv_stream(nnc_hip_kv* kv) { return kv ? static_cast<void*>(kv->stream) : nullptr; }

nnc_status nnc_hip_fill_normal(void* dst, uint64_t n, uint64_t seed, int32_t norm_dim, bool bf16, void* stream)
{
	if (!dst && n) return fail(NNC_ERR_INVALID_ARGUMENT, "NULL destination");
	if (norm_dim < 0 || (norm_dim > 0 && n % static_cast<uint64_t>(norm_dim) != 0))
		return fail(NNC_ERR_INVALID_ARGUMENT, "%llu elements are not whole runs of %d", static_cast<unsigned long long>(n),
		            norm_dim);
	if (n == 0) return NNC_OK;
	nnchip::launch_fill_normal(dst, n, seed, norm_dim, bf16, static_cast<hipStream_t>(stream));
	NNC_HIP_TRY(hipGetLastError(), "fill");
	return NNC_OK;
}

const char* nnc_hip_last_error(void) { return g_last_error.c_str(); }

const char* nnc_hip_status_string(nnc_status status)
{
	switch (status)
	{
	case NNC_OK: return "ok";
	case NNC_ERR_INVALID_ARGUMENT: return "invalid argument";
	case NNC_ERR_UNSUPPORTED_CPU: return "unsupported CPU";
	case NNC_ERR_IO: return "I/O error";
	case NNC_ERR_BAD_FORMAT: return "bad file format";
	case NNC_ERR_UNSUPPORTED_MODEL: return "unsupported model";
	case NNC_ERR_OUT_OF_MEMORY: return "out of memory";
	case NNC_ERR_CONTEXT_FULL: return "context full";
	case NNC_ERR_CANCELLED: return "cancelled";
	}
	return "unknown status";
}

} // extern "C"
