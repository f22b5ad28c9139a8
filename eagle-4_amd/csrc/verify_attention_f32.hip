// Tree-verify attention on fp32 tensors: fp32 q / k_new / v_new / out over fp32 paged caches (vllm/verify_attention.py
// :29-207 computes the same rows for any dtype; the reference runs its own tests on fp32 tensors on the CPU).
//
// The 16-bit schedules' structure at fp32 width, on v_mfma_f32_16x16x4f32:
//  * one workgroup per (context split, KV head, group of four 16-row tiles, request); a row is (draft token, query
//    head of the KV head's group), so every K / V tile read serves G W rows; splits are context chunks (256 keys,
//    fewer for grids too small to fill the chip), the last one also takes the draft keys (masked by the rows'
//    ancestor bits); a request with several splits leaves fp32 partials with their log2-sum-exp, merged by a second
//    kernel (kernels/online_softmax.py:11-24 and vllm/verify_attention.py:115-139);
//  * 16-key tiles staged in LDS — K row-major (pitch D + 4 floats), V transposed to [d][key] (pitch 20 floats), both
//    conflict-free for the 16-byte operand reads — the next tile held in registers while the current one computes;
//  * S^T = K Q^T: block kb of the MFMA contracts over d = g D / 4 + kb for lane group g, so a lane's K and Q operands
//    are D / 4 consecutive floats; the scores land one query row per lane column (4 lanes per row), O^T = V^T P^T
//    takes P^T straight from them (block kb over keys 4 g + kb) and V^T from 16-byte reads of the transposed tile.
// Roofline: the KV read at 4 bytes per element; the fp32 MFMA work (2 D flops per key per row, twice) is below the
// fp32 matrix ridge (~20 flop/B) for the tree widths of a verify, so it is a stream like the 16-bit path.

#include "attention_tile.h"

namespace e4attn {

namespace {

constexpr int kKeysF = 16;  // keys per tile
constexpr int kTilesF = 4;  // 16-row tiles (waves) per workgroup

E4_DEV f32x4_t mma4(float a, float b, f32x4_t c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

template <int D>
struct TileF {
  static constexpr int KP = D + 4;       // K row pitch (floats)
  static constexpr int VP = kKeysF + 4;  // V^T row pitch (floats)
  static constexpr int Q4 = kKeysF * D / 4;  // float4 of one matrix
  static constexpr int PER = (Q4 + 255) / 256;  // float4 per thread per matrix
};

struct ReqF {
  int64_t start;
  int width, context, splits;
};

E4_DEV ReqF req_f(const eagle4_attn_args& a, int b, int chunk) {
  ReqF r;
  r.start = e4::ld(a.query_start_loc, b);
  const int64_t w = e4::ld(a.query_start_loc, b + 1) - r.start;
  r.width = static_cast<int>(w < 64 ? (w < 0 ? 0 : w) : 64);
  int64_t c = e4::ld(a.context_lens, b);
  const int64_t capacity = static_cast<int64_t>(a.max_blocks) * a.page;
  c = c < 0 ? 0 : (c > capacity ? capacity : c);
  r.context = static_cast<int>(c);
  r.splits = c > 0 ? static_cast<int>((c + chunk - 1) / chunk) : 1;
  return r;
}

// One workgroup: kTilesF waves of 16 rows; split blockIdx.x of request blockIdx.z, KV head and row group blockIdx.y.
template <int D>
__global__ __launch_bounds__(64 * kTilesF) void verify_f32_kernel(const eagle4_attn_args a, int chunk, int row_tiles,
                                                                 int max_splits) {
  using TL = TileF<D>;
  __shared__ __attribute__((aligned(16))) float sK[kKeysF * TL::KP];
  __shared__ __attribute__((aligned(16))) float sVt[D * TL::VP];

  const int split = blockIdx.x;
  const int G = a.Hq / a.Hkv;
  const int kvh = blockIdx.y % a.Hkv, rgroup = blockIdx.y / a.Hkv;
  const int b = blockIdx.z;
  const ReqF rq = req_f(a, b, chunk);
  if (split >= rq.splits || rq.width <= 0) return;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, c = lane & 15;
  const int rows = rq.width < a.max_query_len ? rq.width : a.max_query_len;
  const int rt = rgroup * kTilesF + wave;
  const int rho = rt * 16 + c;  // this lane column's query row
  const int t = rho / G, gq = rho % G;
  const bool row_ok = rt < row_tiles && t < rows;
  const int64_t head = static_cast<int64_t>(kvh) * G + gq;
  const float scale_log2 = a.scale * 1.4426950408889634f;

  // Q as the B operand of S^T: q[d = g D / 4 + kb], scaled into the log2 domain
  float q[D / 4];
  {
    const float* qr = static_cast<const float*>(a.q) + (rq.start + (row_ok ? t : 0)) * a.stride_qt + head * a.stride_qh +
                      g * (D / 4);
#pragma unroll
    for (int e = 0; e < D / 16; ++e) {
      const float4 v = row_ok ? *reinterpret_cast<const float4*>(qr + 4 * e) : make_float4(0.f, 0.f, 0.f, 0.f);
      q[4 * e] = v.x * scale_log2;
      q[4 * e + 1] = v.y * scale_log2;
      q[4 * e + 2] = v.z * scale_log2;
      q[4 * e + 3] = v.w * scale_log2;
    }
  }
  const int64_t row_mask = row_ok ? a.masks[b * a.stride_mask + t] : 0;

  const int lo = split * chunk;
  const int hi = lo + chunk < rq.context ? lo + chunk : rq.context;
  const bool has_new = split == rq.splits - 1;
  const int n_ctx = hi > lo ? (hi - lo + kKeysF - 1) / kKeysF : 0;
  const int n_tiles = n_ctx + (has_new ? (rq.width + kKeysF - 1) / kKeysF : 0);

  const float* kc = static_cast<const float*>(a.key_cache) + kvh * a.stride_kh;
  const float* vc = static_cast<const float*>(a.value_cache) + kvh * a.stride_vh;
  const float* kn = static_cast<const float*>(a.k_new) + rq.start * a.stride_knt + kvh * a.stride_knh;
  const float* vn = static_cast<const float*>(a.v_new) + rq.start * a.stride_vnt + kvh * a.stride_vnh;
  const int32_t* bt = static_cast<const int32_t*>(a.block_table.ptr) + b * a.block_table.s0;

  // a tile's K / V rows into registers: float4 e = tid + 256 i is key e / (D / 4), d 4 (e % (D / 4)); keys past the
  // split (or the draft rows) read the last valid one, masked later
  f32x4_t rk[TL::PER], rv[TL::PER];  // native vectors: an array of them stays in registers
  auto load = [&](int tile) {
    const bool is_new = tile >= n_ctx;
#pragma unroll
    for (int i = 0; i < TL::PER; ++i) {
      const int e = tid + 256 * i;
      if (e < TL::Q4) {
        const int kk = e / (D / 4), d4 = 4 * (e % (D / 4));
        const float *ks, *vs;
        if (is_new) {
          const int j0 = (tile - n_ctx) * kKeysF + kk;
          const int64_t j = j0 < rq.width ? j0 : rq.width - 1;
          ks = kn + j * a.stride_knt;
          vs = vn + j * a.stride_vnt;
        } else {
          const int p0 = lo + tile * kKeysF + kk;
          const int pos = p0 < hi ? p0 : hi - 1;
          const int64_t blk = bt[pos / a.page];
          const int64_t sl = pos % a.page;
          ks = kc + blk * a.stride_kb + sl * a.stride_ks;
          vs = vc + blk * a.stride_vb + sl * a.stride_vs;
        }
        rk[i] = *reinterpret_cast<const f32x4_t*>(ks + d4);
        rv[i] = *reinterpret_cast<const f32x4_t*>(vs + d4);
      }
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < TL::PER; ++i) {
      const int e = tid + 256 * i;
      if (e < TL::Q4) {
        const int kk = e / (D / 4), d4 = 4 * (e % (D / 4));
        *reinterpret_cast<f32x4_t*>(sK + kk * TL::KP + d4) = rk[i];
        sVt[(d4 + 0) * TL::VP + kk] = rv[i].x;
        sVt[(d4 + 1) * TL::VP + kk] = rv[i].y;
        sVt[(d4 + 2) * TL::VP + kk] = rv[i].z;
        sVt[(d4 + 3) * TL::VP + kk] = rv[i].w;
      }
    }
  };

  f32x4_t acc[D / 16];  // O^T: acc[dt][r] is d = 16 dt + 4 g + r of row c
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  if (n_tiles > 0) load(0);
  for (int tile = 0; tile < n_tiles; ++tile) {
    __syncthreads();  // the previous tile is no longer read
    stage();
    __syncthreads();
    if (tile + 1 < n_tiles) load(tile + 1);
    const bool is_new = tile >= n_ctx;
    const int base = is_new ? (tile - n_ctx) * kKeysF : lo + tile * kKeysF;

    f32x4_t s = {0.f, 0.f, 0.f, 0.f};  // S^T: s[r] is key 4 g + r of row c
    const float* kr = sK + c * TL::KP + g * (D / 4);
#pragma unroll
    for (int e = 0; e < D / 16; ++e) {
      const float4 k4 = *reinterpret_cast<const float4*>(kr + 4 * e);
      s = mma4(k4.x, q[4 * e], s);
      s = mma4(k4.y, q[4 * e + 1], s);
      s = mma4(k4.z, q[4 * e + 2], s);
      s = mma4(k4.w, q[4 * e + 3], s);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = base + 4 * g + r;
      const bool ok = is_new ? (key < rq.width && ((row_mask >> key) & 1)) : key < hi;
      s[r] = ok ? s[r] : -INFINITY;
      tmax = fmaxf(tmax, s[r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m, tmax);
    const float safe = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m - safe);
    float p[4], psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = exp2f(s[r] - safe);
      psum += p[r];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l = l * alpha + psum;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      const float4 v4 = *reinterpret_cast<const float4*>(sVt + (16 * dt + c) * TL::VP + 4 * g);
      f32x4_t o = acc[dt] * alpha;
      o = mma4(v4.x, p[0], o);
      o = mma4(v4.y, p[1], o);
      o = mma4(v4.z, p[2], o);
      o = mma4(v4.w, p[3], o);
      acc[dt] = o;
    }
  }

  if (!row_ok) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  if (rq.splits == 1) {
    float* orow = static_cast<float*>(a.out) + (rq.start + t) * a.stride_ot + head * a.stride_oh;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
      *reinterpret_cast<float4*>(orow + 16 * dt + 4 * g) =
          make_float4(acc[dt][0] * inv, acc[dt][1] * inv, acc[dt][2] * inv, acc[dt][3] * inv);
  } else {
    const int nrow = row_tiles * 16;
    const int64_t part = ((static_cast<int64_t>(b) * a.Hkv + kvh) * max_splits + split) * nrow + rho;
    store_partial<D>(a.workspace + part * D, acc, inv, g);
    if (g == 0) {
      float* lse = a.workspace + static_cast<int64_t>(a.num_reqs) * a.Hkv * max_splits * nrow * D;
      lse[part] = l > 0.f ? m + log2f(l) : -INFINITY;
    }
  }
}

// The splits of a row merged (vllm/verify_attention.py:115-139): weights 2^(lse_s - max) over the normalised
// partials; one thread per 4 consecutive d of a row.
template <int D>
__global__ __launch_bounds__(256) void verify_f32_merge(const eagle4_attn_args a, int chunk, int row_tiles,
                                                        int max_splits) {
  constexpr int TPR = D / 4;
  constexpr int RPB = 256 / TPR;
  const int b = blockIdx.z, kvh = blockIdx.y;
  const ReqF rq = req_f(a, b, chunk);
  if (rq.splits <= 1 || rq.width <= 0) return;
  const int rho = blockIdx.x * RPB + threadIdx.x / TPR, d = 4 * (threadIdx.x % TPR);
  const int G = a.Hq / a.Hkv;
  const int rows = rq.width < a.max_query_len ? rq.width : a.max_query_len;
  const int t = rho / G, gq = rho % G;
  if (rho >= row_tiles * 16 || t >= rows) return;
  const int nrow = row_tiles * 16;
  const float* lse = a.workspace + static_cast<int64_t>(a.num_reqs) * a.Hkv * max_splits * nrow * D;
  const int64_t part0 = (static_cast<int64_t>(b) * a.Hkv + kvh) * max_splits * nrow + rho;
  // The splits in groups of kMergeGroup, every load of a group issued before the first is used (one memory round trip
  // per group, not per split; a group's loads past the last split re-read the first), the same operations in the same
  // order as one split at a time.
  const int ns = rq.splits;
  float mx = -INFINITY;
  for (int s0 = 0; s0 < ns; s0 += kMergeGroup) {
    float l[kMergeGroup];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i) l[i] = lse[part0 + static_cast<int64_t>(s0 + i < ns ? s0 + i : s0) * nrow];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i)
      if (s0 + i < ns) mx = fmaxf(mx, l[i]);
  }
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  float wsum = 0.f;
  if (mx != -INFINITY) {
    for (int s0 = 0; s0 < ns; s0 += kMergeGroup) {
      float l[kMergeGroup];
      float4 v[kMergeGroup];
#pragma unroll
      for (int i = 0; i < kMergeGroup; ++i) {
        const int64_t part = part0 + static_cast<int64_t>(s0 + i < ns ? s0 + i : s0) * nrow;
        l[i] = lse[part];
        v[i] = *reinterpret_cast<const float4*>(a.workspace + part * D + d);
      }
#pragma unroll
      for (int i = 0; i < kMergeGroup; ++i) {
        if (s0 + i >= ns) break;
        const float w = exp2f(l[i] - mx);
        sum.x += w * v[i].x;
        sum.y += w * v[i].y;
        sum.z += w * v[i].z;
        sum.w += w * v[i].w;
        wsum += w;
      }
    }
  }
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
  *reinterpret_cast<float4*>(static_cast<float*>(a.out) + (rq.start + t) * a.stride_ot +
                             (static_cast<int64_t>(kvh) * G + gq) * a.stride_oh + d) =
      make_float4(sum.x * inv, sum.y * inv, sum.z * inv, sum.w * inv);
}

struct PlanF {
  int chunk, row_tiles, row_groups, max_splits;
};

// Context keys per split: a caller's choice, else 256, shortened (to 128, 48) while the grid of (request, KV head, row
// group) workgroups is too small to occupy the chip (batch 1, L 512, D 128: splits of 32 / 48 / 64 keys 23.8 / 21.8 /
// 24.6 us with the merge).
PlanF plan_f(const eagle4_attn_args& a) {
  PlanF p;
  p.row_tiles = e4::ceil_div(static_cast<int64_t>(a.Hq / a.Hkv) * a.max_query_len, 16);
  p.row_groups = e4::ceil_div(p.row_tiles, kTilesF);
  const int64_t groups = static_cast<int64_t>(a.num_reqs) * a.Hkv * p.row_groups;
  p.chunk = a.chunk > 0 ? a.chunk : (groups < 64 ? 48 : (groups < 256 ? 128 : 256));
  const int64_t capacity = static_cast<int64_t>(a.max_blocks) * a.page;
  p.max_splits = capacity > 0 ? e4::ceil_div(capacity, p.chunk) : 1;
  return p;
}

template <int D>
int launch_f(const eagle4_attn_args& a, const PlanF& p, hipStream_t s) {
  const dim3 grid(p.max_splits, a.Hkv * p.row_groups, a.num_reqs);
  verify_f32_kernel<D><<<grid, 64 * kTilesF, 0, s>>>(a, p.chunk, p.row_tiles, p.max_splits);
  if (p.max_splits > 1) {
    constexpr int RPB = 256 / (D / 4);
    const dim3 mgrid(e4::ceil_div(p.row_tiles * 16, RPB), a.Hkv, a.num_reqs);
    verify_f32_merge<D><<<mgrid, 256, 0, s>>>(a, p.chunk, p.row_tiles, p.max_splits);
  }
  return E4_LAUNCH_STATUS();
}

}  // namespace

// fp32 rows over fp32 pages; 16-byte accesses along D (strides multiples of 4 elements); a caller's split a multiple
// of the 16-key tile; the rest of the contract is checked by the caller.
bool f32_covered(const eagle4_attn_args& a) {
  return a.dtype == EAGLE4_F32 && a.cache_dtype == EAGLE4_F32 && a.chunk >= 0 && a.chunk % kKeysF == 0 &&
         ((a.stride_qt | a.stride_qh | a.stride_knt | a.stride_knh | a.stride_vnt | a.stride_vnh | a.stride_ot |
           a.stride_oh | a.stride_kb | a.stride_ks | a.stride_kh | a.stride_vb | a.stride_vs | a.stride_vh) %
          4) == 0;
}

int64_t f32_workspace_bytes(const eagle4_attn_args& a) {
  const PlanF p = plan_f(a);
  if (p.max_splits <= 1) return 0;
  const int64_t parts = static_cast<int64_t>(a.num_reqs) * a.Hkv * p.max_splits * p.row_tiles * 16;
  return parts * (a.D + 1) * static_cast<int64_t>(sizeof(float));
}

int f32_launch(const eagle4_attn_args& a, hipStream_t s) {
  const PlanF p = plan_f(a);
  if (p.max_splits > 1 && (a.workspace == nullptr || a.workspace_bytes < f32_workspace_bytes(a)))
    return EAGLE4_NOT_COVERED;
  switch (a.D) {
    case 32: return launch_f<32>(a, p, s);
    case 64: return launch_f<64>(a, p, s);
    case 128: return launch_f<128>(a, p, s);
    default: return launch_f<256>(a, p, s);
  }
}

}  // namespace e4attn
