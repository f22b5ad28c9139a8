// What a tree round leaves behind, put back into chain order for vLLM on gfx950 (vllm/round_commit.py): the KV of the
// accepted rows moves to the chain slots context + j in every full-attention layer (KvCompactor, :33-143), and the
// round's rows are rewritten for the draft's prefill (chainize, :146-215).
//
// KV compaction is a gather of at most W - 1 rows of 2 head_dim elements per (request, layer, KV head): one wave per
// triple, each lane a 16-byte chunk of a row. Row j's source is row path[j] >= j (rows are parent first), so no row
// is read after an earlier move wrote it: the moves go in groups of kMoves with every read of a group issued before
// its writes (one memory round trip per group, not per row), which lands the same bytes as the reference's ordered
// loop.

#include "common.h"

namespace {

constexpr int kMoves = 8;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // an array of it stays in registers

// _is_tree (:26-29): more than one query row, one logit per row
E4_DEV bool is_tree(const eagle4_itab& qsl, const eagle4_itab& cu, int b, int64_t& start, int64_t& width) {
  start = e4::ld(qsl, b);
  width = e4::ld(qsl, b + 1) - start;
  return width > 1 && width == e4::ld(cu, b + 1) - e4::ld(cu, b);
}

// _compact_kv_kernel (:33-83): one wave per (KV head, layer, request). `vec`: the host found the cache strides and
// the row length multiples of 16 bytes; each layer's base is checked here.
__global__ __launch_bounds__(64) void compact_kv_kernel(const eagle4_compact_kv_args a, int vec) {
  const int head = blockIdx.x, layer = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  int64_t start, width;
  if (!is_tree(a.query_start_loc, a.cu_num_logits, b, start, width)) return;
  const int64_t slot = e4::ld(a.idx_mapping, b);
  const int64_t context = e4::ld(a.seq_lens, b) - width;
  const int64_t n = e4::ld(a.path_len, slot);
  char* const base = reinterpret_cast<char*>(a.layer_ptrs[layer]);
  const int32_t* const table = reinterpret_cast<const int32_t*>(a.table_ptrs[layer]) + b * a.table_strides[layer];
  const int64_t tbs = a.table_block_sizes[layer];
  // byte offset of the row of token position `pos` of the request (:65-77)
  auto at = [&](int64_t pos) {
    const int64_t token = static_cast<int64_t>(table[pos / tbs]) * tbs + pos % tbs;
    const int64_t blk = token / a.block_size, in = token % a.block_size;
    return 2 * (blk * a.stride_block + head * a.stride_head + in * a.stride_slot);
  };
  const bool v16 = vec && (reinterpret_cast<uintptr_t>(base) & 15) == 0;
  const int units = v16 ? a.dim / 8 : a.dim;  // 16-byte chunks, or 2-byte elements, of a row
  for (int64_t j0 = 1; j0 < n; j0 += kMoves) {
    int64_t src[kMoves], dst[kMoves];
    bool move[kMoves];
#pragma unroll
    for (int i = 0; i < kMoves; ++i) {
      const int64_t j = j0 + i;
      const int64_t s = j < n ? context + e4::ld(a.path, slot, j) : context + j;
      move[i] = j < n && s != context + j;
      src[i] = move[i] ? at(s) : 0;
      dst[i] = move[i] ? at(context + j) : 0;
    }
    for (int u = lane; u < units; u += 64) {
      if (v16) {
        u32x4 val[kMoves];
#pragma unroll
        for (int i = 0; i < kMoves; ++i)
          if (move[i]) val[i] = *reinterpret_cast<const u32x4*>(base + src[i] + 16 * u);
#pragma unroll
        for (int i = 0; i < kMoves; ++i)
          if (move[i]) *reinterpret_cast<u32x4*>(base + dst[i] + 16 * u) = val[i];
      } else {
        uint16_t val[kMoves];
#pragma unroll
        for (int i = 0; i < kMoves; ++i)
          if (move[i]) val[i] = *reinterpret_cast<const uint16_t*>(base + src[i] + 2 * u);
#pragma unroll
        for (int i = 0; i < kMoves; ++i)
          if (move[i]) *reinterpret_cast<uint16_t*>(base + dst[i] + 2 * u) = val[i];
      }
    }
  }
}

E4_DEV void store_int(void* p, int64_t i, int dtype, int64_t v) {
  if (dtype == EAGLE4_I64)
    static_cast<int64_t*>(p)[i] = v;
  else
    static_cast<int32_t*>(p)[i] = static_cast<int32_t>(v);
}

// _chainize_kernel (:146-179): one wave per request, lane r its row r (< rows, the stage width's power of two).
__global__ __launch_bounds__(64) void chainize_kernel(const eagle4_chainize_args a) {
  const int b = blockIdx.x, r = threadIdx.x;
  int64_t start, width;
  if (!is_tree(a.query_start_loc, a.cu_num_logits, b, start, width)) return;
  if (r >= a.rows || r >= width) return;
  const int64_t slot = e4::ld(a.idx_mapping, b);
  const int64_t pl = e4::ld(a.path_len, slot);
  const int64_t accepted = pl < width ? pl : width;
  const int64_t context = e4::ld(a.seq_lens, b) - width;
  // row r takes the hidden state of accepted row path[r] (rows past the path keep their own), position context + r
  const int64_t src = r < accepted ? e4::ld(a.path, slot, r) : r;
  store_int(a.src_rows, start + r, a.src_rows_dtype, start + src);
  store_int(a.positions, start + r, a.positions_dtype, context + r);
  // and the sampled token r - 1 (row 0 keeps the root's)
  if (r >= 1 && r < accepted) store_int(a.input_ids, start + r, a.input_ids_dtype, e4::ld(a.sampled, b, r - 1));
}

bool tab_ok(const eagle4_itab& t) { return t.ptr != nullptr && e4::is_index_dtype(t.dtype); }

}  // namespace

extern "C" int eagle4_compact_kv(const eagle4_compact_kv_args* a, void* stream) {
  if (a->num_reqs == 0 || a->layers == 0 || a->heads == 0) return EAGLE4_OK;
  if (a->layer_ptrs == nullptr || a->table_ptrs == nullptr || a->table_strides == nullptr ||
      a->table_block_sizes == nullptr || !tab_ok(a->idx_mapping) || !tab_ok(a->query_start_loc) ||
      !tab_ok(a->cu_num_logits) || !tab_ok(a->seq_lens) || !tab_ok(a->path) || !tab_ok(a->path_len) ||
      (a->dtype != EAGLE4_BF16 && a->dtype != EAGLE4_F16) || a->dim <= 0 || a->block_size <= 0 ||
      a->num_reqs > 65535 || a->layers > 65535)
    return EAGLE4_NOT_COVERED;
  const int vec = (a->dim % 8 == 0 && a->stride_block % 8 == 0 && a->stride_head % 8 == 0 && a->stride_slot % 8 == 0)
                      ? 1
                      : 0;
  const dim3 grid(a->heads, a->layers, a->num_reqs);
  compact_kv_kernel<<<grid, 64, 0, static_cast<hipStream_t>(stream)>>>(*a, vec);
  return E4_LAUNCH_STATUS();
}

extern "C" int eagle4_chainize(const eagle4_chainize_args* a, void* stream) {
  if (a->num_reqs == 0) return EAGLE4_OK;
  const auto int_ok = [](int d) { return d == EAGLE4_I32 || d == EAGLE4_I64; };
  if (!tab_ok(a->idx_mapping) || !tab_ok(a->query_start_loc) || !tab_ok(a->cu_num_logits) || !tab_ok(a->seq_lens) ||
      !tab_ok(a->path) || !tab_ok(a->path_len) || !tab_ok(a->sampled) || a->input_ids == nullptr ||
      a->positions == nullptr || a->src_rows == nullptr || !int_ok(a->input_ids_dtype) ||
      !int_ok(a->positions_dtype) || !int_ok(a->src_rows_dtype) || a->rows < 1 || a->rows > 64)
    return EAGLE4_NOT_COVERED;
  chainize_kernel<<<a->num_reqs, 64, 0, static_cast<hipStream_t>(stream)>>>(*a);
  return E4_LAUNCH_STATUS();
}
