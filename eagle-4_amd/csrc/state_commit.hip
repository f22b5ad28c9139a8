// vLLM's accepted-path commit of the linear-attention state on gfx950 (vllm/gdn_tree_verify.py:186-322): the window
// columns of the accepted rows move next to each other and the recurrent state of the last accepted row moves into
// the slot the next round resumes from, for every layer, in one launch.
//
// One grid, two roles by workgroup index: the first workgroups compact the windows (a block of 256 channels, 128 for
// fp32 windows, of one request and layer each), the rest move states (a 64 KB chunk of one request's slot and layer
// each), so the small window work runs beside the state copies instead of as a launch of its own.
//
// Window compaction (_compact_window_kernel, :185-215). The reference moves column 2 + path[j] to 2 + j in ascending
// j. A root path is increasing (rows are parent first), so path[j] >= j: a column read at step j is either never
// written or written at a later step, and every read sees the column's value from before the commit. The moves of a
// block therefore run as one gather: every (channel, j) source is read (consecutive threads take consecutive j of a
// channel, then the next channel: dense, mostly contiguous addresses), the workgroup synchronises, every destination
// is written.
//
// State move (_move_state_kernel, :218-245): a pure HBM copy of 2 x HV V K elements per moved request and layer,
// 16-byte loads and stores, every load of a thread issued before its stores.

#include "common.h"

namespace {

constexpr int64_t kNullBlock = 0;
constexpr int kThreads = 256;
// channels per window workgroup: the gathered values of a block take 32 KB of LDS
template <typename S>
constexpr int kChannels = sizeof(S) == 2 ? 256 : 128;
constexpr int kMaxMoves = 63;     // window moves per channel (trees of up to 64 rows)
constexpr int kCopies = 16;       // 16-byte copies in flight per thread
constexpr int64_t kChunk = 16 * kCopies * kThreads;  // state bytes per workgroup

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // an array of it stays in registers

struct CommitPlan {
  int64_t win_groups;  // workgroups [0, win_groups) compact windows
  int win_blocks;      // channel blocks per (request, layer)
  int state_chunks;    // chunks per slot
};

template <typename S>
__device__ void compact_window(const eagle4_state_commit_args& a, int64_t id, int blocks, S* s_val) {
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
  const int items = nch * m;
  for (int i = threadIdx.x; i < items; i += kThreads) {
    const int ch = i / m, j = 1 + i % m;
    const int64_t src = 2 + e4::ld(a.path, state, j);
    s_val[i] = base[ch * a.conv_stride_dim + src * a.conv_stride_tok];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < items; i += kThreads) {
    const int ch = i / m, j = 1 + i % m;
    if (e4::ld(a.path, state, j) != j) base[ch * a.conv_stride_dim + (2 + j) * a.conv_stride_tok] = s_val[i];
  }
}

__device__ void move_state(const eagle4_state_commit_args& a, int64_t id, int chunks) {
  const int64_t rl = id / chunks;
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
  const int64_t lo = (id % chunks) * kChunk;
  const int64_t hi = lo + kChunk < bytes ? lo + kChunk : bytes;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | bytes) & 15) == 0) {
    for (int64_t i0 = lo + threadIdx.x * 16; i0 < hi; i0 += 16 * kCopies * kThreads) {
      u32x4 v[kCopies];
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int64_t i = i0 + static_cast<int64_t>(c) * 16 * kThreads;
        if (i < hi) v[c] = *(const __attribute__((address_space(1))) u32x4*)reinterpret_cast<uintptr_t>(src + i);
      }
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int64_t i = i0 + static_cast<int64_t>(c) * 16 * kThreads;
        if (i < hi) *(__attribute__((address_space(1))) u32x4*)reinterpret_cast<uintptr_t>(dst + i) = v[c];
      }
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += kThreads) dst[i] = src[i];
  }
}

template <typename S>
__global__ __launch_bounds__(kThreads) void commit_kernel(const eagle4_state_commit_args a, const CommitPlan p) {
  __shared__ S s_val[kChannels<S> * kMaxMoves];
  const int64_t id = blockIdx.x;
  if (id < p.win_groups)
    compact_window<S>(a, id, p.win_blocks, s_val);
  else
    move_state(a, id - p.win_groups, p.state_chunks);
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
  const int channels = a->conv_dtype == EAGLE4_F32 ? kChannels<float> : kChannels<uint16_t>;
  p.win_blocks = a->dim > 0 ? e4::ceil_div(a->dim, channels) : 0;
  p.win_groups = static_cast<int64_t>(p.win_blocks) * a->num_reqs * a->layers;
  const int esize = a->ssm_dtype == EAGLE4_F32 ? 4 : 2;
  p.state_chunks = a->ssm_numel > 0 ? e4::ceil_div(a->ssm_numel * esize, kChunk) : 0;
  const int64_t groups = p.win_groups + static_cast<int64_t>(p.state_chunks) * a->num_reqs * a->layers;
  if (groups == 0) return EAGLE4_OK;
  if (a->conv_dtype == EAGLE4_F32)
    commit_kernel<float><<<static_cast<unsigned>(groups), kThreads, 0, s>>>(*a, p);
  else  // 16-bit windows: a raw copy either way
    commit_kernel<uint16_t><<<static_cast<unsigned>(groups), kThreads, 0, s>>>(*a, p);
  return E4_LAUNCH_STATUS();
}
