// vLLM's accepted-path commit of the linear-attention state on gfx950 (vllm/gdn_tree_verify.py:186-322): the window
// columns of the accepted rows move next to each other and the recurrent state of the last accepted row moves into
// the slot the next round resumes from, for every layer, in one launch.
//
// One grid, two roles by workgroup index: the first workgroups move states (about 1024 of them, each a contiguous
// split of one request's slot and layer), the rest compact the windows (a block of 256 channels, 128 for fp32
// windows, of one request and layer each), so the small window work fills the end of the state copies instead of
// running as a launch of its own.
//
// Window compaction (_compact_window_kernel, :185-215). The reference moves column 2 + path[j] to 2 + j in ascending
// j. A root path is increasing (rows are parent first), so path[j] >= j: a column read at step j is either never
// written or written at a later step, and every read sees the column's value from before the commit. The moves of a
// block therefore run as one gather from a copy of the block taken before any write. When a slot's rows are
// contiguous (token stride 1: the block is one span of kChannels x row-stride elements) the span is copied into LDS
// with 16-byte direct loads and written back in 16-byte pieces, each assembled from the copy, a piece only when one
// of its columns moves; otherwise every (channel, j) source is read element-wise into LDS and the destinations are
// written element-wise.
//
// State move (_move_state_kernel, :218-245): a pure HBM copy of 2 x HV V K elements per moved request and layer,
// 16-byte loads and stores, both with the nontemporal policy: the source (the walk's snapshot of the accepted node)
// is read once (batch-64 step 0.775 -> 0.771 ms), and the moved states leave no dirty lines in the last-level cache
// for the next step's kernels to write back (0.767 -> 0.756 ms: the walk that reads them as its initial states
// 438 -> 421 us in the step). A workgroup looks its request's slots up once and copies its split in 32 KB steps, two
// steps in flight, so the lookups' latency is paid once per split rather than once per step.

#include "common.h"

namespace {

constexpr int64_t kNullBlock = 0;
constexpr int kThreads = 256;
// channels per window workgroup (a span of 9.5 KB at the 16-bit, 19-column windows of 16-node trees)
template <typename S>
constexpr int kChannels = sizeof(S) == 2 ? 256 : 128;
constexpr int kMaxMoves = 63;     // window moves per channel (trees of up to 64 rows)
constexpr int kCopies = 8;        // 16-byte loads per thread per step (two steps in flight)
constexpr int64_t kStep = 16 * kCopies * kThreads;  // 32 KB of state per step
constexpr int64_t kStateGroups = 1024;             // state workgroups aimed at (4 per CU), whatever the batch

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // an array of it stays in registers

struct CommitPlan {
  int64_t state_groups;  // workgroups [0, state_groups) move states, the rest compact windows
  int64_t split_bytes;   // state bytes per state workgroup (a multiple of the step)
  int splits;            // state workgroups per (request, layer)
  int win_blocks;        // channel blocks per (request, layer)
  int lds_bytes;         // a window workgroup's LDS for the span or the gathered values (the source columns follow)
};

// 64 lanes x 16 bytes from per-lane global addresses into LDS [dst, dst + 1024), lane p at dst + 16 p.
E4_DEV void dma16(const void* src, char* dst) { __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0); }

// The window compaction of one (request, layer, channel block). `lds` holds `lds_bytes` bytes: the block's span
// (span form) or a pass of gathered values (element form), then the moves' source columns.
template <typename S>
__device__ void compact_window(const eagle4_state_commit_args& a, int64_t id, int blocks, int lds_bytes, char* lds) {
  const int cb = static_cast<int>(id % blocks);
  const int64_t rl = id / blocks;
  const int b = static_cast<int>(rl % a.num_reqs), layer = static_cast<int>(rl / a.num_reqs);
  const int64_t state = e4::ld(a.idx_mapping, b);
  const int32_t* slots = reinterpret_cast<const int32_t*>(a.slots_ptrs[layer]);
  const int64_t slot = slots[b * a.slots_strides[layer]];
  const int n = static_cast<int>(e4::ld(a.path_len, state));
  if (slot <= kNullBlock || n <= 1) return;
  const int m = n - 1 < kMaxMoves ? n - 1 : kMaxMoves;  // moves per channel: j = 1 .. m
  const int ch0 = cb * kChannels<S>;
  const int nch = a.dim - ch0 < kChannels<S> ? a.dim - ch0 : kChannels<S>;
  S* base = reinterpret_cast<S*>(a.conv_ptrs[layer]) + slot * a.conv_stride_slot + ch0 * a.conv_stride_dim;
  const int tid = threadIdx.x;
  int* const s_src = reinterpret_cast<int*>(lds + lds_bytes);  // [1 + kMaxMoves]: source column of column 2 + j
  for (int j = 1 + tid; j <= m; j += kThreads) s_src[j] = 2 + static_cast<int>(e4::ld(a.path, state, j));
  // the span form: token stride 1, rows of conv_stride_dim elements, a 16-byte aligned block that fits the LDS
  constexpr int kPer = 16 / sizeof(S);  // elements per 16-byte piece
  const int rowlen = static_cast<int>(a.conv_stride_dim);
  const int pieces = nch * rowlen / kPer;
  if (a.conv_stride_tok == 1 && (reinterpret_cast<uintptr_t>(base) & 15) == 0 && (nch * rowlen) % kPer == 0 &&
      pieces * 16 <= lds_bytes) {
    for (int k = tid >> 6; k * 64 < pieces; k += kThreads / 64) {  // 1 KB per direct load; past the end: the last
      const int i = k * 64 + (tid & 63) < pieces ? k * 64 + (tid & 63) : pieces - 1;
      dma16(reinterpret_cast<const char*>(base) + 16 * static_cast<int64_t>(i), lds + k * 1024);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the direct loads have landed in LDS
    __syncthreads();
    const S* old = reinterpret_cast<const S*>(lds);
    for (int i = tid; i < pieces; i += kThreads) {
      union {
        uint4 v;
        S e[kPer];
      } piece;
      piece.v = reinterpret_cast<const uint4*>(old)[i];
      bool moved = false;
      int c = (i * kPer) / rowlen, col = i * kPer - c * rowlen;
#pragma unroll
      for (int e = 0; e < kPer; ++e) {
        const int j = col - 2;
        if (j >= 1 && j <= m) {
          const int src = s_src[j];
          if (src != col) {
            piece.e[e] = old[c * rowlen + src];
            moved = true;
          }
        }
        if (++col == rowlen) {
          col = 0;
          ++c;
        }
      }
      if (moved) reinterpret_cast<uint4*>(base)[i] = piece.v;
    }
    return;
  }
  // the element form, in passes of as many channels as the LDS holds
  __syncthreads();
  S* s_val = reinterpret_cast<S*>(lds);
  const int per = lds_bytes / static_cast<int>(sizeof(S)) / m;
  for (int c0 = 0; c0 < nch; c0 += per) {
    const int items = (nch - c0 < per ? nch - c0 : per) * m;
    for (int i = tid; i < items; i += kThreads) {
      const int ch = c0 + i / m, j = 1 + i % m;
      s_val[i] = base[ch * a.conv_stride_dim + s_src[j] * a.conv_stride_tok];
    }
    __syncthreads();
    for (int i = tid; i < items; i += kThreads) {
      const int ch = c0 + i / m, j = 1 + i % m;
      if (s_src[j] != 2 + j) base[ch * a.conv_stride_dim + (2 + j) * a.conv_stride_tok] = s_val[i];
    }
    __syncthreads();
  }
}

// State move of one (request, layer, split): bytes [part x split_bytes, + split_bytes) of the accepted row's slot into
// the slot the next round resumes from. 32 KB steps, the next step's loads issued before the current step's stores,
// so every thread keeps 16 loads in flight.
__device__ void move_state(const eagle4_state_commit_args& a, int64_t id, int splits, int64_t split_bytes) {
  const int64_t rl = id / splits;
  const int b = static_cast<int>(rl % a.num_reqs), layer = static_cast<int>(rl / a.num_reqs);
  const int64_t state = e4::ld(a.idx_mapping, b);
  const int64_t length = e4::ld(a.path_len, state);
  const int64_t last = e4::ld(a.path, state, length - 1);
  const int32_t* slots = reinterpret_cast<const int32_t*>(a.slots_ptrs[layer]) + b * a.slots_strides[layer];
  const int64_t src_slot = slots[last];
  const int64_t dst_slot = slots[length - 1];
  if (!(last != length - 1 && src_slot > kNullBlock && dst_slot > kNullBlock)) return;
  const int esize = a.ssm_dtype == EAGLE4_F32 ? 4 : 2;
  const char* src = reinterpret_cast<const char*>(a.ssm_ptrs[layer]) + src_slot * a.ssm_stride_slot * esize;
  char* dst = reinterpret_cast<char*>(a.ssm_ptrs[layer]) + dst_slot * a.ssm_stride_slot * esize;
  const int64_t bytes = a.ssm_numel * esize;
  const int64_t lo = (id % splits) * split_bytes;
  const int64_t hi = lo + split_bytes < bytes ? lo + split_bytes : bytes;
  const int tid = threadIdx.x;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | bytes) & 15) == 0) {
    typedef __attribute__((address_space(1))) const u32x4 gsrc;
    typedef __attribute__((address_space(1))) u32x4 gdst;
    auto load = [&](u32x4 (&v)[kCopies], int64_t i0) {
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int64_t i = i0 + (static_cast<int64_t>(c) * kThreads + tid) * 16;
        if (i < hi) v[c] = __builtin_nontemporal_load(reinterpret_cast<gsrc*>(reinterpret_cast<uintptr_t>(src + i)));
      }
    };
    auto store = [&](const u32x4 (&v)[kCopies], int64_t i0) {
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int64_t i = i0 + (static_cast<int64_t>(c) * kThreads + tid) * 16;
        if (i < hi) __builtin_nontemporal_store(v[c], reinterpret_cast<gdst*>(reinterpret_cast<uintptr_t>(dst + i)));
      }
    };
    u32x4 v0[kCopies], v1[kCopies];
    int64_t i0 = lo;
    if (i0 < hi) load(v0, i0);
    while (i0 < hi) {  // two steps per pass, the buffers alternating
      const int64_t i1 = i0 + kStep;
      if (i1 < hi) load(v1, i1);
      store(v0, i0);
      if (i1 >= hi) break;
      const int64_t i2 = i1 + kStep;
      if (i2 < hi) load(v0, i2);
      store(v1, i1);
      i0 = i2;
    }
  } else {
    for (int64_t i = lo + tid; i < hi; i += kThreads) dst[i] = src[i];
  }
}

template <typename S>
__global__ __launch_bounds__(kThreads) void commit_kernel(const eagle4_state_commit_args a, const CommitPlan p) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int64_t id = blockIdx.x;
  if (id < p.state_groups)
    move_state(a, id, p.splits, p.split_bytes);
  else
    compact_window<S>(a, id - p.state_groups, p.win_blocks, p.lds_bytes, lds);
}

bool tab_ok(const eagle4_itab& t) { return t.ptr != nullptr && e4::is_index_dtype(t.dtype); }

}  // namespace

extern "C" int eagle4_linear_state_commit(const eagle4_state_commit_args* a, void* stream) {
  if (a->num_reqs == 0 || a->layers == 0) return EAGLE4_OK;
  if (!tab_ok(a->idx_mapping) || !tab_ok(a->path) || !tab_ok(a->path_len) || a->conv_ptrs == nullptr ||
      a->ssm_ptrs == nullptr || a->slots_ptrs == nullptr || a->slots_strides == nullptr ||
      !e4::is_float_dtype(a->conv_dtype) || !e4::is_float_dtype(a->ssm_dtype))
    return EAGLE4_NOT_COVERED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  CommitPlan p;
  const bool f32 = a->conv_dtype == EAGLE4_F32;
  const int channels = f32 ? kChannels<float> : kChannels<uint16_t>;
  const int esz_conv = f32 ? 4 : 2;
  p.win_blocks = a->dim > 0 ? e4::ceil_div(a->dim, channels) : 0;
  const int64_t win_groups = static_cast<int64_t>(p.win_blocks) * a->num_reqs * a->layers;
  const int esize = a->ssm_dtype == EAGLE4_F32 ? 4 : 2;
  const int64_t pairs = static_cast<int64_t>(a->num_reqs) * a->layers;
  const int64_t state_bytes = a->ssm_numel * esize;
  p.splits = 0;
  p.split_bytes = kStep;
  if (state_bytes > 0) {  // about kStateGroups workgroups, each a whole number of steps
    const int64_t want = e4::ceil_div(kStateGroups, pairs);
    p.split_bytes = e4::ceil_div(e4::ceil_div(state_bytes, want), kStep) * kStep;
    p.splits = static_cast<int>(e4::ceil_div(state_bytes, p.split_bytes));
  }
  p.state_groups = static_cast<int64_t>(p.splits) * pairs;
  // a window block's LDS: its span (rows of conv_stride_dim elements) when that is at most 32 KB, else 32 KB
  const int64_t span_bytes = static_cast<int64_t>(channels) * a->conv_stride_dim * esz_conv;
  p.lds_bytes = static_cast<int>(span_bytes <= 32 * 1024 ? e4::ceil_div(span_bytes, 1024) * 1024 : 32 * 1024);
  if (p.lds_bytes < 16 * kMaxMoves) p.lds_bytes = 16 * kMaxMoves;  // one channel's moves at least, 16-byte multiple
  const int64_t groups = p.state_groups + win_groups;
  if (groups == 0) return EAGLE4_OK;
  const size_t lds = static_cast<size_t>(p.lds_bytes) + 4 * (1 + kMaxMoves);
  if (f32)
    commit_kernel<float><<<static_cast<unsigned>(groups), kThreads, lds, s>>>(*a, p);
  else  // 16-bit windows: a raw copy either way
    commit_kernel<uint16_t><<<static_cast<unsigned>(groups), kThreads, lds, s>>>(*a, p);
  return E4_LAUNCH_STATUS();
}
