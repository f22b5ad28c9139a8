// vLLM's accepted-path commit of the linear-attention state on gfx950 (vllm/gdn_tree_verify.py:186-322): the window
// columns of the accepted rows move next to each other and the recurrent state of the last accepted row moves into
// the slot the next round resumes from, for every layer in one launch each.
//
// The state move is a pure HBM copy (2 x 2 MB per request and layer at HV = 32, K = V = 128, fp32): 16-byte loads and
// stores, a grid of (chunks, requests, layers) with the chunks sized so a launch has thousands of workgroups.

#include "common.h"

namespace {

constexpr int64_t kNullBlock = 0;

// _compact_window_kernel (:185-215): one thread per channel of (request, layer). The reference moves column
// 2 + path[j] to 2 + j in ascending j; since path[j] >= j, no column is read after an earlier step wrote it, so the
// moves are made kMoves at a time with every read of a group issued before its writes (one memory round trip per
// group instead of one per column).
template <typename T>
__global__ __launch_bounds__(128) void compact_window_kernel(const eagle4_state_commit_args a) {
  using S = typename T::storage;
  constexpr int kMoves = 8;
  const int b = blockIdx.x, layer = blockIdx.y;
  const int f = blockIdx.z * blockDim.x + threadIdx.x;
  if (f >= a.dim) return;
  const int64_t state = e4::ld(a.idx_mapping, b);
  const int32_t* slots = reinterpret_cast<const int32_t*>(a.slots_ptrs[layer]);
  const int64_t slot = slots[b * a.slots_strides[layer]];
  if (slot <= kNullBlock) return;
  S* base = reinterpret_cast<S*>(a.conv_ptrs[layer]) + slot * a.conv_stride_slot + f * a.conv_stride_dim;
  const int64_t n = e4::ld(a.path_len, state);
  for (int64_t j0 = 1; j0 < n; j0 += kMoves) {
    int64_t src[kMoves];
    S val[kMoves];
#pragma unroll
    for (int i = 0; i < kMoves; ++i) src[i] = j0 + i < n ? 2 + e4::ld(a.path, state, j0 + i) : 2 + j0 + i;
#pragma unroll
    for (int i = 0; i < kMoves; ++i)
      if (src[i] != 2 + j0 + i) val[i] = base[src[i] * a.conv_stride_tok];
#pragma unroll
    for (int i = 0; i < kMoves; ++i)
      if (src[i] != 2 + j0 + i) base[(2 + j0 + i) * a.conv_stride_tok] = val[i];
  }
}

// _move_state_kernel (:218-245): blockIdx.x walks kCopies x 16-byte chunks per thread of the slot, every load of a
// thread issued before its stores (the pools are device memory: global loads and stores, not flat ones).
constexpr int kCopies = 16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // an array of it stays in registers

__global__ __launch_bounds__(256) void move_state_kernel(const eagle4_state_commit_args a, int64_t chunk_bytes) {
  const int b = blockIdx.y, layer = blockIdx.z;
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
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * chunk_bytes;
  const int64_t hi = lo + chunk_bytes < bytes ? lo + chunk_bytes : bytes;
  if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | bytes) & 15) == 0) {
    for (int64_t i0 = lo + threadIdx.x * 16; i0 < hi; i0 += 16 * kCopies * blockDim.x) {
      u32x4 v[kCopies];
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int64_t i = i0 + static_cast<int64_t>(c) * 16 * blockDim.x;
        if (i < hi) v[c] = *(const __attribute__((address_space(1))) u32x4*)reinterpret_cast<uintptr_t>(src + i);
      }
#pragma unroll
      for (int c = 0; c < kCopies; ++c) {
        const int64_t i = i0 + static_cast<int64_t>(c) * 16 * blockDim.x;
        if (i < hi) *(__attribute__((address_space(1))) u32x4*)reinterpret_cast<uintptr_t>(dst + i) = v[c];
      }
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) dst[i] = src[i];
  }
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
  if (a->dim > 0) {
    const dim3 grid(a->num_reqs, a->layers, e4::ceil_div(a->dim, 128));
    if (a->conv_dtype == EAGLE4_F32)
      compact_window_kernel<e4::F32><<<grid, 128, 0, s>>>(*a);
    else
      compact_window_kernel<e4::Bf16><<<grid, 128, 0, s>>>(*a);  // 16-bit: a raw copy either way
  }
  if (a->ssm_numel > 0) {
    const int esize = a->ssm_dtype == EAGLE4_F32 ? 4 : 2;
    constexpr int64_t kChunk = 16 * kCopies * 256;  // per workgroup: kCopies x 16-byte copies per thread
    const int64_t bytes = a->ssm_numel * esize;
    const dim3 grid(e4::ceil_div(bytes, kChunk), a->num_reqs, a->layers);
    move_state_kernel<<<grid, 256, 0, s>>>(*a, kChunk);
  }
  return E4_LAUNCH_STATUS();
}
