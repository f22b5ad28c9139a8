// Tree tables of a verify round on gfx950: the verify stage (depths, window codes, ancestor masks, depth positions),
// the link -> parent derivation with the conv window codes and the path table, and the tail-mask words.
//
// These are integer and launch-latency bound (a few hundred bytes per request). One workgroup per request: one lane
// runs the serial parent-first recurrence over the rows in LDS (every row reads rows before it), then the wave writes
// the rows out in parallel.

#include "common.h"

namespace {

constexpr int kStageMaxWidth = 64;

// vllm/verify_layout.py:31-86 (_stage_tree_kernel), with VerifyStage.stage's save of the chain positions (:159)
// folded in: each request's workgroup copies its own rows' positions before rewriting them (and the last one the
// tokens after the last request), so no separate copy launch runs.
//
// Lane u holds row u. A parent-first tree (0 <= parent(u) < u for 0 < u < W: every tree the drafter builds) is
// staged by pointer jumping over lane shuffles: depths and ancestor-or-self masks accumulate along the jumps (at
// most six rounds for 64 rows), the window codes are the parent, grandparent and great-grandparent read directly.
// Anything else replays the reference's serial update order on one lane, so every input stages as the reference
// stages it.
__global__ __launch_bounds__(64) void stage_tree_kernel(const eagle4_stage_tree_args a) {
  __shared__ int32_t s_par[kStageMaxWidth], s_depth[kStageMaxWidth];
  __shared__ int32_t s_anc1[kStageMaxWidth], s_anc2[kStageMaxWidth], s_anc3[kStageMaxWidth];
  __shared__ int64_t s_mask[kStageMaxWidth];
  const int b = blockIdx.x;
  const int lane = threadIdx.x;
  const int W = a.width;
  const int WP = W <= 1 ? 1 : (1 << (32 - __clz(W - 1)));
  // one round of independent table loads, then the request's parents and positions together
  const int64_t slot = e4::ld(a.idx_mapping, b);
  const int64_t start = e4::ld(a.query_start_loc, b);
  const int64_t width = e4::ld(a.query_start_loc, b + 1) - start;
  const int64_t logits = e4::ld(a.cu_num_logits, b + 1) - e4::ld(a.cu_num_logits, b);
  const bool is_tree = a.tree && width > 1 && width == logits;  // :54
  const int32_t loaded = lane < W ? static_cast<int32_t>(e4::ld(a.parents, slot, lane)) : -1;  // :57
  const int64_t pos = lane < width ? a.positions[start + lane] : 0;
  const int64_t pos0 = width > 0 ? __shfl(pos, 0, 64) : a.positions[start];  // :52 reads it for any width
  if (a.chain_positions != nullptr) {  // the saved chain positions: this request's rows, before the rewrite below
    if (lane < width) a.chain_positions[start + lane] = pos;
    for (int64_t i = start + 64 + lane; i < start + width; i += 64) a.chain_positions[i] = a.positions[i];
    if (b == 0) {  // the tokens before the first request
      for (int64_t i = lane; i < start; i += 64) a.chain_positions[i] = a.positions[i];
    }
    if (b == a.num_reqs - 1) {  // the tokens after the last request
      for (int64_t i = start + width + lane; i < a.num_tokens; i += 64) a.chain_positions[i] = a.positions[i];
    }
  }
  const int par = is_tree ? loaded : lane - 1;  // :59 (lanes past W: -1 from the load, or a chain's lane - 1)
  const bool parent_first = __ballot(lane > 0 && lane < W && (par < 0 || par >= lane)) == 0;
  int depth = 0, anc1 = -1, anc2 = -2, anc3 = -3;
  int64_t mask = 1;
  if (parent_first) {
    const bool row = lane > 0 && lane < W;
    int up = row ? par : lane;                    // the root and lanes past W point at themselves
    depth = row ? 1 : 0;
    // every row descends from the root: its bit 0 is set from the start (a jump that reaches the root stops the
    // loop before the root's own mask would be read)
    mask = row ? ((static_cast<int64_t>(1) << lane) | 1) : (lane == 0 ? 1 : 0);
    for (int r = 0; r < 6 && __ballot(row && up != 0) != 0; ++r) {
      const int d2 = __shfl(depth, up, 64);
      const int64_t m2 = __shfl(mask, up, 64);
      const int u2 = __shfl(up, up, 64);
      depth += d2;
      mask |= m2;
      up = u2;
    }
    const int p1 = __shfl(par, row ? par : 0, 64);  // the parent's parent (row 0's -1 for a child of the root)
    const int p2 = __shfl(par, row && p1 > 0 ? p1 : 0, 64);
    if (row) {
      anc1 = par;
      anc2 = par == 0 ? -1 : p1;            // anc1 of the parent: the root's is -1
      anc3 = par == 0 ? -2 : (p1 == 0 ? -1 : p2);  // anc2 of the parent
    }
  } else {
    if (lane < WP) {
      s_par[lane] = par;
      s_depth[lane] = 0;
      s_anc1[lane] = -1;
      s_anc2[lane] = -2;
      s_anc3[lane] = -3;
      s_mask[lane] = 1;
    }
    __syncthreads();
    if (lane == 0) {
      // :66-74 in the kernel's update order; a parent outside [0, WP) reads zeros, like the masked vector sums
      for (int r = 1; r < W; ++r) {
        const int p = s_par[r];
        const bool in = p >= 0 && p < WP;
        s_depth[r] = (in ? s_depth[p] : 0) + 1;
        s_anc1[r] = p;
        s_anc2[r] = in ? s_anc1[p] : 0;
        s_anc3[r] = in ? s_anc2[p] : 0;
        s_mask[r] = (in ? s_mask[p] : 0) | (static_cast<int64_t>(1) << r);
      }
    }
    __syncthreads();
    if (lane < W) {
      depth = s_depth[lane];
      anc1 = s_anc1[lane];
      anc2 = s_anc2[lane];
      anc3 = s_anc3[lane];
      mask = s_mask[lane];
    }
  }
  if (lane == 0) a.context_lens[b] = static_cast<int32_t>(pos0);  // :52
  if (lane < W) {
    const int64_t out = static_cast<int64_t>(b) * W + lane;
    a.stage_parents[out] = par;
    a.stage_anc[static_cast<int64_t>(b) * 3 * W + lane] = anc1;
    a.stage_anc[static_cast<int64_t>(b) * 3 * W + W + lane] = anc2;
    a.stage_anc[static_cast<int64_t>(b) * 3 * W + 2 * W + lane] = anc3;
    a.stage_mask[out] = mask;
    a.slot_parents[slot * W + lane] = par;
    a.slot_depths[slot * W + lane] = depth;
    if (is_tree && lane < width) a.positions[start + lane] = pos - lane + depth;  // :85-86: context + depth
  }
}

constexpr int kAncMaxWidth = 1024;

// kernels/gdn_tree.py:44-89 (_gdn_tree_paths), on the parents in LDS (NP entries). Lane-parallel parts run on all
// threads of the block; the serial depth pass runs on thread 0.
__device__ void build_paths(int32_t* s_par_in, int32_t* s_tmp, int32_t* s_packed, int NP, int num_tokens, int seqlen,
                            int32_t* paths, int64_t stride_path) {
  const int tid = threadIdx.x;
  for (int i = tid; i < NP; i += blockDim.x) {  // :57-61 sanitised parents
    const int p = s_par_in[i];
    s_tmp[i] = (i > 0 && p >= 0 && p < i) ? p : (i > 0 ? i - 1 : 0);
    s_packed[i] = 0;
  }
  __syncthreads();
  if (tid == 0) {
    for (int t = 1; t < seqlen; ++t) {  // :64-72
      const int p = s_tmp[t];
      const int pp = (p >= 0 && p < NP) ? s_packed[p] : 0;
      const int depth = (pp & 255) + 1;
      const int chain_depth = pp >= 65536 ? depth : ((pp >> 8) & 255);
      if (t < num_tokens) {
        s_packed[t] = depth + (chain_depth << 8);
        if (p >= 0 && p < NP) s_packed[p] |= 65536;
      }
    }
  }
  __syncthreads();
  // leaf ranks: an exclusive count of the leaves before each node (:74-76), serial over <= 256 nodes
  __shared__ int32_t s_rank[256];
  __shared__ int32_t s_num_leaves;
  if (tid == 0) {
    int rank = 0;
    for (int i = 0; i < NP; ++i) {
      const bool leaf = i < num_tokens && s_packed[i] < 65536;
      s_rank[i] = leaf ? rank : -1;
      rank += leaf ? 1 : 0;
    }
    s_num_leaves = rank;
  }
  __syncthreads();
  const int num_leaves = s_num_leaves;
  for (int i = tid; i < NP; i += blockDim.x) {
    const int r = s_rank[i];
    if (r >= 0) {
      int32_t* row = paths + static_cast<int64_t>(r) * stride_path;
      const int depth = s_packed[i] & 255;
      row[0] = depth + 1;                   // :78
      row[1] = (s_packed[i] >> 8) & 255;    // :79
      int node = i;                         // :86-89, leaf first
      for (int step = 0; step <= depth; ++step) {
        row[2 + depth - step] = node;
        node = (node >= 0 && node < NP) ? s_tmp[node] : 0;
      }
    }
  }
  for (int i = tid; i < seqlen; i += blockDim.x) {  // :80-84: the length column of the rows past the leaf count
    if (i >= num_leaves) paths[static_cast<int64_t>(i) * stride_path] = 0;
  }
}

// kernels/gdn_tree.py:93-186 (_gdn_tree_ancestors_kernel).
__global__ __launch_bounds__(256) void ancestors_kernel(const eagle4_ancestors_args a) {
  __shared__ int32_t s_next[kAncMaxWidth], s_sib[kAncMaxWidth], s_par[kAncMaxWidth];
  __shared__ int32_t s_a1[kAncMaxWidth], s_a2[kAncMaxWidth], s_a3[kAncMaxWidth];
  const int seq = blockIdx.x;
  const int tid = threadIdx.x;
  const int width = a.width;
  const int NP = width <= 1 ? 1 : (1 << (32 - __clz(width - 1)));
  const int64_t coord = e4::ld(a.conv_state_indices, seq);
  int num_tokens = 0;
  if (a.paths != nullptr) {
    int64_t n = e4::ld(a.query_start_loc, seq + 1) - e4::ld(a.query_start_loc, seq);
    n = n < 0 ? 0 : n;
    num_tokens = static_cast<int>(n < width ? n : width);  // :123-126
  }
  int32_t* paths = a.paths == nullptr ? nullptr : a.paths + static_cast<int64_t>(seq) * a.stride_paths_seq;
  if (coord == a.pad_slot_id) {  // :127-138: padded rows keep their parents; their paths follow them
    if (paths != nullptr) {
      for (int i = tid; i < NP; i += blockDim.x)
        s_par[i] = i < width ? static_cast<int32_t>(e4::ld(a.parent_token, seq, i)) : 0;
      __syncthreads();
      build_paths(s_par, s_a1, s_a2, NP, num_tokens, width, paths, a.stride_paths_path);
    }
    return;
  }
  for (int i = tid; i < NP; i += blockDim.x) {
    s_next[i] = i < width ? static_cast<int32_t>(e4::ld(a.next_token, seq, i)) : -1;
    s_sib[i] = i < width ? static_cast<int32_t>(e4::ld(a.next_sibling, seq, i)) : -1;
    s_par[i] = 0;
    s_a1[i] = -1;
    s_a2[i] = -2;
    s_a3[i] = -3;
  }
  __syncthreads();
  if (tid == 0) {  // :155-172, the upstream derivation order
    for (int t = 0; t < width; ++t) {
      const int n = s_next[t];
      if (n != -1 && n >= 0 && n < NP) s_par[n] = t;
      const int sib = s_sib[t];
      const int p = s_par[t];
      if (sib != -1 && sib >= 0 && sib < NP) s_par[sib] = p;
      int g = (p >= 0 && p < NP) ? s_par[p] : 0;
      g = p > 0 ? g : p - 1;
      int gg = (g >= 0 && g < NP) ? s_par[g] : 0;
      gg = g > 0 ? gg : g - 1;
      if (t > 0) {
        s_a1[t] = p;
        s_a2[t] = g;
        s_a3[t] = gg;
      }
    }
  }
  __syncthreads();
  int32_t* anc = a.ancestors + static_cast<int64_t>(seq) * 3 * width;
  for (int i = tid; i < width; i += blockDim.x) {
    e4::st(a.parent_token, seq, i, s_par[i]);
    anc[i] = s_a1[i];
    anc[width + i] = s_a2[i];
    anc[2 * width + i] = s_a3[i];
  }
  if (paths != nullptr) {
    __syncthreads();
    build_paths(s_par, s_a1, s_a2, NP, num_tokens, width, paths, a.stride_paths_path);
  }
}

// kernels/verify_prep.py:23-33 (_tail_words_kernel): lane r packs row r's tail bits.
__global__ __launch_bounds__(64) void tail_words_kernel(const eagle4_tail_words_args a) {
  const int r = threadIdx.x;
  const int64_t kv_len = e4::ld(a.committed_len, 0) + a.width;
  if (r < a.width) {
    uint64_t bits = 0;
    const uint8_t* row = a.mask + static_cast<int64_t>(r) * kv_len + (kv_len - a.width);
    for (int j = 0; j < a.width; ++j) bits |= static_cast<uint64_t>(row[j] != 0) << j;
    a.tail_bits[r] = static_cast<int64_t>(bits);
  }
}

bool tab_ok(const eagle4_itab& t) { return t.ptr != nullptr && e4::is_index_dtype(t.dtype); }

}  // namespace

extern "C" int eagle4_stage_tree(const eagle4_stage_tree_args* a, void* stream) {
  if (a->num_reqs == 0) return EAGLE4_OK;
  if (a->width < 1 || a->width > kStageMaxWidth || !tab_ok(a->parents) || !tab_ok(a->idx_mapping) ||
      !tab_ok(a->query_start_loc) || !tab_ok(a->cu_num_logits))
    return EAGLE4_NOT_COVERED;
  stage_tree_kernel<<<a->num_reqs, 64, 0, static_cast<hipStream_t>(stream)>>>(*a);
  return E4_LAUNCH_STATUS();
}

extern "C" int eagle4_gdn_tree_ancestors(const eagle4_ancestors_args* a, void* stream) {
  if (a->batch == 0) return EAGLE4_OK;
  if (a->width < 1 || a->width > kAncMaxWidth || !tab_ok(a->next_token) || !tab_ok(a->next_sibling) ||
      !tab_ok(a->parent_token) || !tab_ok(a->conv_state_indices))
    return EAGLE4_NOT_COVERED;
  if (a->paths != nullptr && (a->width >= 256 || !tab_ok(a->query_start_loc))) return EAGLE4_NOT_COVERED;
  ancestors_kernel<<<a->batch, 256, 0, static_cast<hipStream_t>(stream)>>>(*a);
  return E4_LAUNCH_STATUS();
}

extern "C" int eagle4_tree_tail_words(const eagle4_tail_words_args* a, void* stream) {
  if (a->width < 1 || a->width > 64 || !tab_ok(a->committed_len)) return EAGLE4_NOT_COVERED;
  tail_words_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(*a);
  return E4_LAUNCH_STATUS();
}
