// Greedy acceptance of a verified tree on gfx950: the target's argmax per row, the tree walk, the bs1 accept tail
// and the row compaction (vllm/tree_accept.py:45-115, kernels/accept_tail.py:56-224).
//
// The argmax is the HBM-bound part (the logits of every verify row, 2.49 GB at 8192 x 151936 bf16): one workgroup
// per row streams it with 16-byte loads and reduces (max, first index) in registers, then across the block. The walk
// and the tail are a few hundred bytes per request, one thread per request.

#include "common.h"

namespace {

// (value, index) with the first index on ties (torch.argmax); NaN compares as the largest value.
E4_DEV bool better(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

template <typename T>
__global__ __launch_bounds__(256) void argmax_kernel(const eagle4_argmax_args a) {
  using S = typename T::storage;
  const int row = blockIdx.x;
  const S* p = static_cast<const S*>(a.logits) + static_cast<int64_t>(row) * a.stride_row;
  constexpr int VEC = 16 / sizeof(S);
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
  const bool aligned = (reinterpret_cast<uintptr_t>(p) % 16) == 0;
  const int nvec = aligned ? a.vocab / VEC : 0;
  // UNR 16-byte loads in flight per thread before any is reduced (a thread's vectors are v, v + 256, ...; positions
  // past the row re-read its first vector and are skipped)
  constexpr int UNR = 4;
  for (int v0 = threadIdx.x; v0 < nvec; v0 += UNR * blockDim.x) {
    uint4 raw[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int v = v0 + u * static_cast<int>(blockDim.x);
      {  // read once, nontemporally: the 2.5 GB of logits do not churn the last-level cache (449 -> 397 us at 8192 rows)
        typedef uint32_t u32x4n __attribute__((ext_vector_type(4)));
        const u32x4n t =
            __builtin_nontemporal_load(reinterpret_cast<const u32x4n*>(p + static_cast<int64_t>(v < nvec ? v : 0) * VEC));
        raw[u] = make_uint4(t.x, t.y, t.z, t.w);
      }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int v = v0 + u * static_cast<int>(blockDim.x);
      const S* e = reinterpret_cast<const S*>(&raw[u]);
      float f[VEC];
#pragma unroll
      for (int i = 0; i < VEC; ++i) f[i] = T::to_f32(e[i]);
      // the vector's max (NaN-ignoring) and sum (NaN when a NaN, or opposite infinities, is in it): only a vector
      // that can change the thread's best — a larger value, a NaN, or the thread's first vector — is searched
      float m = f[0], sum = f[0];
#pragma unroll
      for (int i = 1; i < VEC; ++i) {
        m = fmaxf(m, f[i]);
        sum += f[i];
      }
      if (v < nvec && (m > bv || sum != sum || bi == INT64_MAX)) {
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          const int64_t idx = static_cast<int64_t>(v) * VEC + i;
          if (better(f[i], idx, bv, bi)) {
            bv = f[i];
            bi = idx;
          }
        }
      }
    }
  }
  for (int64_t i = static_cast<int64_t>(nvec) * VEC + threadIdx.x; i < a.vocab; i += blockDim.x) {
    const float f = T::to_f32(p[i]);
    if (better(f, i, bv, bi)) {
      bv = f;
      bi = i;
    }
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int64_t oi = __shfl_xor(bi, m, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float s_v[4];
  __shared__ int64_t s_i[4];
  if ((threadIdx.x & 63) == 0) {
    s_v[threadIdx.x >> 6] = bv;
    s_i[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w)
      if (better(s_v[w], s_i[w], bv, bi)) {
        bv = s_v[w];
        bi = s_i[w];
      }
    a.out[row] = bi;
  }
}

// vllm/tree_accept.py:45-83 (_tree_accept_kernel): one thread per request.
__global__ void accept_tree_kernel(const eagle4_accept_tree_args a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.num_reqs) return;
  const int64_t slot = e4::ld(a.idx_mapping, b);
  const int64_t start = e4::ld(a.cu_num_logits, b);
  const int64_t rows = e4::ld(a.cu_num_logits, b + 1) - start;
  const int64_t limit = rows < a.width ? rows : a.width;
  int node = 0, count = 0;
  bool alive = rows > 0;
  for (int step = 0; step < a.width; ++step) {
    if (!alive) break;
    const int64_t token = e4::ld(a.target, start + node);
    a.sampled[b * a.stride_sampled + step] = token;
    a.path[slot * a.stride_path + step] = node;
    ++count;
    int child = -1;
    for (int r = 1; r < limit; ++r) {  // the lowest-index row that continues the walk (:78-79)
      if (e4::ld(a.parents, slot, r) == node && e4::ld(a.drafted, start + r) == token) {
        child = r;
        break;
      }
    }
    alive = child >= 0;
    if (alive) node = child;
  }
  a.num_sampled[b] = count;
  a.path_len[slot] = count;
}

// kernels/accept_tail.py:56-132 (_accept_tail_kernel), batch size 1. The walk down the tree is serial (one thread), a
// chain of dependent lookups, so its tables are first read by the 64 lanes at once into LDS (entries 0-63: a tree of at
// most 64 rows; any other index is read from global memory), and the outputs are written by the lanes in parallel
// after it (8.8 -> 4.8 us at width 16).
__global__ __launch_bounds__(64) void accept_tail_kernel(const eagle4_accept_tail_args a) {
  constexpr int N = 64;
  __shared__ int64_t s_ri[N], s_nt[N], s_ns[N], s_cand[N], s_tp[N];
  __shared__ int32_t s_acc[N];
  __shared__ int64_t s_num, s_last;
  const int t = threadIdx.x;
  const int width = a.width, depth = a.depth;
  const int n = width < N ? width : N;
  if (t < n) {
    s_ri[t] = e4::ld(a.retrieve_index, t);
    s_nt[t] = e4::ld(a.retrieve_next_token, t);
    s_ns[t] = e4::ld(a.retrieve_next_sibling, t);
    s_cand[t] = e4::ld(a.candidates, t);
    s_tp[t] = e4::ld(a.target_predict, t);
  }
  const int64_t seq_len = e4::ld(a.seq_lens, 0);
  const int64_t row = e4::ld(a.req_pool_indices, 0);
  __syncthreads();
  auto get = [&](const int64_t* lds, const eagle4_itab& tab, int64_t i) {
    return i >= 0 && i < n ? lds[i] : e4::ld(tab, i);
  };
  if (t == 0) {
    for (int d = 0; d < depth && d < N; ++d) s_acc[d] = -1;  // :79-80
    int64_t last = get(s_ri, a.retrieve_index, 0);
    if (depth > 0) s_acc[0] = static_cast<int32_t>(last);
    int64_t cur = 0, num = 0;
    bool active = true;
    for (int level = 1; level < depth && active; ++level) {  // :90-106
      cur = get(s_nt, a.retrieve_next_token, cur);
      const int64_t target_token = get(s_tp, a.target_predict, last);
      int found = 0;
      for (int sibling = 0; sibling < width && found == 0; ++sibling) {
        const bool valid = cur != -1;
        const int64_t safe = valid ? cur : 0;
        const int64_t node = get(s_ri, a.retrieve_index, safe);
        const bool match = valid && get(s_cand, a.candidates, safe) == target_token;
        if (match) {
          if (num + 1 < N) s_acc[num + 1] = static_cast<int32_t>(node);
          num += 1;
          last = node;
        } else if (valid) {
          cur = get(s_ns, a.retrieve_next_sibling, safe);
        }
        found = match ? 1 : (valid ? 0 : -1);
      }
      active = found == 1;
    }
    s_num = num;
    s_last = last;
  }
  __syncthreads();
  const int64_t num = s_num, last = s_last;
  for (int d = t; d < depth; d += N) a.accept_index[d] = d < N ? s_acc[d] : -1;
  if (t == 0) {  // :110-113: accept lengths, the bonus token, the new length
    a.accept_lens[0] = static_cast<int32_t>(num + 1);
    e4::st(eagle4_itab{a.new_seq_lens, 0, 0, a.seq_lens.dtype, 0}, 0, 0, seq_len + num + 1);
    a.bonus[0] = static_cast<int32_t>(get(s_tp, a.target_predict, last));
  }
  // :115-123: the accepted path moved to the front (padding reads node 0's target)
  for (int node = t; node < width; node += N) {
    int64_t value;
    if (node < depth) {
      const int64_t p = node < N ? s_acc[node] : -1;
      value = get(s_tp, a.target_predict, p > 0 ? p : 0);
    } else {
      bool on_path = false;
      for (int d = 0; d < depth && d <= num && d < N; ++d) on_path |= s_acc[d] == node;
      value = on_path ? get(s_tp, a.target_predict, node) : 0;
    }
    a.predict[node] = static_cast<int32_t>(value);
  }
  // :126-132: the KV slots to move
  for (int d = t; d < depth; d += N) {
    const bool keep = d <= num;
    const int64_t acc = d < N ? s_acc[d] : -1;
    a.committed_slots[d] = keep ? e4::ld(a.req_to_token, row, seq_len + d) : 0;
    a.accepted_slots[d] = keep ? e4::ld(a.out_cache_loc, acc) : 0;
  }
}

// kernels/accept_tail.py:190-206 (_compact_rows_kernel), 16-byte chunks when the row bytes allow.
__global__ __launch_bounds__(256) void compact_rows_kernel(const eagle4_compact_rows_args a) {
  const int row = blockIdx.y;
  int64_t src_row = row;
  if (row < a.depth) {
    const int64_t p = e4::ld(a.accept_index, 0, row < a.depth - 1 ? row : a.depth - 1);
    src_row = p > 0 ? p : 0;
  }
  const char* src = static_cast<const char*>(a.src) + src_row * a.src_stride;
  char* dst = static_cast<char*>(a.dst) + static_cast<int64_t>(row) * a.dst_stride;
  const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | a.row_bytes) & 15) == 0;
  if (vec) {
    for (int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 16; i < a.row_bytes;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x * 16)
      *reinterpret_cast<uint4*>(dst + i) = *reinterpret_cast<const uint4*>(src + i);
  } else {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.row_bytes;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
      dst[i] = src[i];
  }
}

bool tab_ok(const eagle4_itab& t) { return t.ptr != nullptr && e4::is_index_dtype(t.dtype); }

}  // namespace

extern "C" int eagle4_argmax_rows(const eagle4_argmax_args* a, void* stream) {
  if (a->rows == 0) return EAGLE4_OK;
  if (a->vocab < 1 || a->out == nullptr) return EAGLE4_NOT_COVERED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->dtype) {
    case EAGLE4_BF16: argmax_kernel<e4::Bf16><<<a->rows, 256, 0, s>>>(*a); break;
    case EAGLE4_F16: argmax_kernel<e4::F16><<<a->rows, 256, 0, s>>>(*a); break;
    case EAGLE4_F32: argmax_kernel<e4::F32><<<a->rows, 256, 0, s>>>(*a); break;
    default: return EAGLE4_NOT_COVERED;
  }
  return E4_LAUNCH_STATUS();
}

extern "C" int eagle4_accept_tree(const eagle4_accept_tree_args* a, void* stream) {
  if (a->num_reqs == 0) return EAGLE4_OK;
  if (!tab_ok(a->target) || !tab_ok(a->drafted) || !tab_ok(a->cu_num_logits) || !tab_ok(a->idx_mapping) ||
      !tab_ok(a->parents) || a->width < 1)
    return EAGLE4_NOT_COVERED;
  accept_tree_kernel<<<e4::ceil_div(a->num_reqs, 64), 64, 0, static_cast<hipStream_t>(stream)>>>(*a);
  return E4_LAUNCH_STATUS();
}

extern "C" int eagle4_accept_tail(const eagle4_accept_tail_args* a, void* stream) {
  if (!tab_ok(a->target_predict) || !tab_ok(a->candidates) || !tab_ok(a->retrieve_index) ||
      !tab_ok(a->retrieve_next_token) || !tab_ok(a->retrieve_next_sibling) || !tab_ok(a->seq_lens) ||
      !tab_ok(a->out_cache_loc) || !tab_ok(a->req_to_token) || !tab_ok(a->req_pool_indices) || a->depth < 0 ||
      a->depth > 64)  // the accepted path is kept in LDS (trees of at most 64 rows: depth <= 64)
    return EAGLE4_NOT_COVERED;
  accept_tail_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(*a);
  return E4_LAUNCH_STATUS();
}

extern "C" int eagle4_compact_rows(const eagle4_compact_rows_args* a, void* stream) {
  if (a->width == 0 || a->row_bytes == 0) return EAGLE4_OK;
  if (!tab_ok(a->accept_index) || a->depth < 1) return EAGLE4_NOT_COVERED;
  const int64_t chunks = (a->row_bytes + 16 * 256 - 1) / (16 * 256);
  const dim3 grid(static_cast<unsigned>(chunks < 64 ? chunks : 64), a->width);
  compact_rows_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(*a);
  return E4_LAUNCH_STATUS();
}
