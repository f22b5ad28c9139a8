// Tree-verify attention on gfx950: GQA rows over a paged (bf16 / f16 / fp8-e4m3) KV cache plus the round's draft
// rows (vllm/verify_attention.py:29-207, kernels/online_softmax.py:11-24).
//
// Roofline: HBM reads of the KV cache (~94 FLOP/B at batch 64, tree width 16, GQA 6, D 256; the bf16 MFMA ridge is
// ~310 FLOP/B). The design reads every KV byte once and keeps the reads in flight:
//
//  * One workgroup per (split of the context, KV head, request). Its NW waves own 16 query rows each, where a row
//    is (draft token, query head of the KV head's group), so all G x W rows of a KV head share one read of every
//    K / V tile (the reference's grid is per query head and re-reads each tile G times).
//  * Splits are fixed-size context chunks; a request uses ceil(L / chunk) of them (the grid is sized for the page
//    table's capacity and idle splits exit at once). The last split also takes the draft keys, masked by the rows'
//    ancestor bits. A request with one split writes its output directly; others write fp32 partials with their
//    log2-sum-exp, merged by a second kernel.
//  * 32-key tiles are staged in LDS: K row-major (row pitch D + 8 elements: conflict-free 16-byte operand reads), V
//    transposed to [d][key] in registers (8x8 16-bit transposes) under an XOR swizzle. A tile's K / V is loaded into
//    registers one tile ahead and its page-table entries two tiles ahead, branch-free, so neither the page lookup
//    nor the HBM read is exposed; fp8 pages are dequantised (x * scale of the (page, KV head)) at the LDS store.
//  * Scores are S^T = K Q^T on v_mfma_f32_16x16x32: a lane then holds one query row's scores (4 lanes per row), so
//    P^T is the B operand of O^T = V^T P^T straight from registers and O^T keeps one row per lane: the online
//    softmax rescale is a per-lane multiply. 16 rows per wave keep O^T at D / 4 VGPRs per lane, leaving room for two
//    workgroups per CU.

#include <type_traits>

#include "attention_tile.h"

namespace {

using namespace e4attn;

struct Req {
  int64_t start, width, context;
  int splits;
};

// A request's rows and context; the context is clamped to what its page-table row can address, so no split, page
// lookup or partial index leaves the tables and the workspace whatever context_lens holds.
E4_DEV Req request_info(const eagle4_attn_args& a, int b, int chunk) {
  Req r;
  r.start = e4::ld(a.query_start_loc, b);
  r.width = e4::ld(a.query_start_loc, b + 1) - r.start;
  r.context = e4::ld(a.context_lens, b);
  const int64_t capacity = static_cast<int64_t>(a.max_blocks) * a.page;
  r.context = r.context < 0 ? 0 : (r.context > capacity ? capacity : r.context);
  const int64_t s = (r.context + chunk - 1) / chunk;
  r.splits = s < 1 ? 1 : static_cast<int>(s);
  return r;
}

// Uniform addressing of one workgroup's (request, KV head) pages: byte bases of its head in the two caches, byte
// strides, its block-table row, and the page size as a shift when it is a power of two.
struct KvAddr {
  const char* kbase;
  const char* vbase;
  int64_t kb, ks, vb, vs;
  const int32_t* bt;
  const float* kscale;  // k_scale + kvh * stride_ksh (fp8)
  const float* vscale;
  int64_t ksb, vsb;
  int page, page_shift;
};

E4_DEV void page_of(const KvAddr& k, int pos, int& blk_idx, int& slot) {
  if (k.page_shift >= 0) {
    blk_idx = pos >> k.page_shift;
    slot = pos & (k.page - 1);
  } else {
    blk_idx = static_cast<int>(static_cast<uint32_t>(pos) / static_cast<uint32_t>(k.page));
    slot = pos - blk_idx * k.page;
  }
}

// The pages of the rows a wave's direct loads fill (instructions n = wave + NW m), looked up two tiles ahead.
template <int D, int NW>
struct DirectPages {
  static constexpr int NIW = (Tile<D>::NI + NW - 1) / NW;
  int blk[NIW], slot[NIW];
};

template <int D, int NW>
E4_DEV void lookup_direct(DirectPages<D, NW>& p, const KvAddr& kv, int base, int hi, int wave, int lane) {
  using TL = Tile<D>;
#pragma unroll
  for (int m = 0; m < DirectPages<D, NW>::NIW; ++m) {
    const int n = wave + NW * m;
    const int pos = base + n * TL::RPI + lane / TL::CH;
    int bi;
    page_of(kv, pos < hi ? pos : hi - 1, bi, p.slot[m]);  // past the split: the split's last key (masked later)
    p.blk[m] = n < TL::NI ? kv.bt[bi] : 0;
  }
}

template <int D, int NW>
E4_DEV void issue_direct_ctx(char* sKb, char* sVb, const DirectPages<D, NW>& p, const KvAddr& kv, int wave, int lane) {
  using TL = Tile<D>;
#pragma unroll
  for (int m = 0; m < DirectPages<D, NW>::NIW; ++m) {
    const int n = wave + NW * m;
    if (n < TL::NI) {
      const int row = n * TL::RPI + lane / TL::CH, pc = lane % TL::CH;
      const int64_t off = static_cast<int64_t>(p.blk[m]) * kv.kb + static_cast<int64_t>(p.slot[m]) * kv.ks;
      const int64_t offv = static_cast<int64_t>(p.blk[m]) * kv.vb + static_cast<int64_t>(p.slot[m]) * kv.vs;
      // the builtin takes its source as a plain pointer variable (a compound expression fails its overload check)
      const char* ksrc = kv.kbase + off + 16 * (pc ^ TL::kswz(row));
      const char* vsrc = kv.vbase + offv + 16 * (pc ^ TL::vswz(row));
      __builtin_amdgcn_global_load_lds(ksrc, sKb + n * 1024, 16, 0, 2);
      __builtin_amdgcn_global_load_lds(vsrc, sVb + n * 1024, 16, 0, 2);
    }
  }
}

// Draft rows (16-bit): row r of the tile is draft key first + r, clamped to the last draft key (masked later).
template <int D, int NW>
E4_DEV void issue_direct_new(char* sKb, char* sVb, const char* knew, const char* vnew, int64_t kstride,
                             int64_t vstride, int first, int width, int wave, int lane) {
  using TL = Tile<D>;
#pragma unroll
  for (int m = 0; m < DirectPages<D, NW>::NIW; ++m) {
    const int n = wave + NW * m;
    if (n < TL::NI) {
      const int row = n * TL::RPI + lane / TL::CH, pc = lane % TL::CH;
      const int key = first + row < width ? first + row : width - 1;
      const char* ksrc = knew + static_cast<int64_t>(key) * kstride + 16 * (pc ^ TL::kswz(row));
      const char* vsrc = vnew + static_cast<int64_t>(key) * vstride + 16 * (pc ^ TL::vswz(row));
      __builtin_amdgcn_global_load_lds(ksrc, sKb + n * 1024, 16, 0, 2);
      __builtin_amdgcn_global_load_lds(vsrc, sVb + n * 1024, 16, 0, 2);
    }
  }
}

// fp8 context tiles: (row, chunk) pairs q = tid + NT i, loaded raw into registers, dequantised into LDS later.
template <int D, int NW>
struct Fp8Tile {
  static constexpr int NT = 64 * NW;
  static constexpr int NQ = (kTileKeys * Tile<D>::CH + NT - 1) / NT;
  uint2 k[NQ], v[NQ];
  float ks[NQ], vs[NQ];
};

template <int D, int NW>
E4_DEV void load_fp8(Fp8Tile<D, NW>& r, const KvAddr& kv, int base, int hi, int tid) {
  using TL = Tile<D>;
  constexpr int NT = 64 * NW;
  int blk[Fp8Tile<D, NW>::NQ], sl[Fp8Tile<D, NW>::NQ];
#pragma unroll
  for (int i = 0; i < Fp8Tile<D, NW>::NQ; ++i) {
    const int q = tid + NT * i;
    const int pos = base + q / TL::CH;
    int bi;
    page_of(kv, pos < hi ? pos : hi - 1, bi, sl[i]);
    blk[i] = q < kTileKeys * TL::CH ? kv.bt[bi] : 0;
  }
#pragma unroll
  for (int i = 0; i < Fp8Tile<D, NW>::NQ; ++i) {
    const int q = tid + NT * i;
    const int lc = q % TL::CH;
    if (q < kTileKeys * TL::CH) {
      const int64_t b = blk[i];
      r.k[i] = *reinterpret_cast<const uint2*>(kv.kbase + b * kv.kb + static_cast<int64_t>(sl[i]) * kv.ks + 8 * lc);
      r.v[i] = *reinterpret_cast<const uint2*>(kv.vbase + b * kv.vb + static_cast<int64_t>(sl[i]) * kv.vs + 8 * lc);
      r.ks[i] = kv.kscale[b * kv.ksb];
      r.vs[i] = kv.vscale[b * kv.vsb];
    }
  }
}

template <int D, int NW, typename T>
E4_DEV void store_fp8(char* sKb, char* sVb, const Fp8Tile<D, NW>& r, int tid) {
  using TL = Tile<D>;
  constexpr int NT = 64 * NW;
#pragma unroll
  for (int i = 0; i < Fp8Tile<D, NW>::NQ; ++i) {
    const int q = tid + NT * i;
    if (q < kTileKeys * TL::CH) {
      const int row = q / TL::CH, lc = q % TL::CH;
      *reinterpret_cast<uint4*>(sKb + row * TL::ROWB + 16 * (lc ^ TL::kswz(row))) = dequant8<T>(r.k[i], r.ks[i]);
      *reinterpret_cast<uint4*>(sVb + row * TL::ROWB + 16 * (lc ^ TL::vswz(row))) = dequant8<T>(r.v[i], r.vs[i]);
    }
  }
}

E4_DEV void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Starts tile `tile`'s K / V towards LDS buffer tile & 1: draft rows and 16-bit pages by direct loads, fp8 pages into
// registers (dequantised and stored after this tile's compute).
template <int D, int NW, typename T, bool FP8>
E4_DEV void issue_tile(int tile, char (*smem)[2][Tile<D>::BYTES], int n_ctx, Fp8Tile<D, NW>& f8,
                       const DirectPages<D, NW>& pages, const KvAddr& kv, int lo, int hi, const char* knp,
                       const char* vnp, int64_t skt, int64_t svt, int width, int tid, int wave, int lane) {
  char* kb = smem[tile & 1][0];
  char* vb = smem[tile & 1][1];
  if (tile >= n_ctx) {
    issue_direct_new<D, NW>(kb, vb, knp, vnp, skt, svt, (tile - n_ctx) * kTileKeys, width, wave, lane);
  } else if constexpr (FP8) {
    load_fp8<D, NW>(f8, kv, lo + tile * kTileKeys, hi, tid);
  } else {
    issue_direct_ctx<D, NW>(kb, vb, pages, kv, wave, lane);
  }
}

template <int D, int NW, typename T, bool FP8>
__global__ __launch_bounds__(64 * NW) void verify_attention_kernel(const eagle4_attn_args a, int chunk, int row_tiles,
                                                                  int max_splits) {
  static_assert(D % 32 == 0 && D >= 32 && D <= 256, "head dim");
  using TL = Tile<D>;
  __shared__ __attribute__((aligned(1024))) char smem[2][2][TL::BYTES];  // [buffer][K, V]

  const int split = blockIdx.x;
  const int G = a.Hq / a.Hkv;
  const int kvh = blockIdx.y % a.Hkv;
  const int rgroup = blockIdx.y / a.Hkv;
  const int b = blockIdx.z;
  const Req rq = request_info(a, b, chunk);
  if (split >= rq.splits || rq.width <= 0) return;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, l16 = lane & 15;
  const int rt = rgroup * NW + wave;
  const bool computes = rt < row_tiles;
  const int rho = rt * 16 + l16;  // this lane's query row
  const int t = rho / G, gq = rho % G;
  const bool row_ok = computes && t < rq.width && t < a.max_query_len;
  const int64_t head = static_cast<int64_t>(kvh) * G + gq;

  uint4 qreg[D / 32];
  load_q<D>(qreg, static_cast<const uint16_t*>(a.q) + (rq.start + t) * a.stride_qt + head * a.stride_qh, row_ok, g);
  const int64_t row_mask = row_ok ? a.masks[b * a.stride_mask + t] : 0;

  f32x4_t acc[D / 16];  // O^T: acc[dt][i] is d = 16 dt + 4 g + i of the lane's row
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float scale_log2 = a.scale * 1.4426950408889634f;

  const int lo = split * chunk;  // context positions stay below 2^31
  const int hi = static_cast<int>(lo + chunk < rq.context ? lo + chunk : rq.context);
  const bool has_new = split == rq.splits - 1;
  const int width = static_cast<int>(rq.width < 64 ? rq.width : 64);
  const int n_ctx = hi > lo ? (hi - lo + kTileKeys - 1) / kTileKeys : 0;
  const int n_tiles = n_ctx + (has_new ? (width + kTileKeys - 1) / kTileKeys : 0);

  KvAddr kv;
  {
    constexpr int EB = FP8 ? 1 : 2;
    kv.kbase = static_cast<const char*>(a.key_cache) + kvh * a.stride_kh * EB;
    kv.vbase = static_cast<const char*>(a.value_cache) + kvh * a.stride_vh * EB;
    kv.kb = a.stride_kb * EB;
    kv.ks = a.stride_ks * EB;
    kv.vb = a.stride_vb * EB;
    kv.vs = a.stride_vs * EB;
    kv.bt = static_cast<const int32_t*>(a.block_table.ptr) + b * a.block_table.s0;
    kv.kscale = FP8 ? a.k_scale + kvh * a.stride_ksh : nullptr;
    kv.vscale = FP8 ? a.v_scale + kvh * a.stride_vsh : nullptr;
    kv.ksb = a.stride_ksb;
    kv.vsb = a.stride_vsb;
    kv.page = a.page;
    kv.page_shift = (a.page & (a.page - 1)) == 0 ? __builtin_ctz(a.page) : -1;
  }
  const char* knp = static_cast<const char*>(a.k_new) + (rq.start * a.stride_knt + kvh * a.stride_knh) * 2;
  const char* vnp = static_cast<const char*>(a.v_new) + (rq.start * a.stride_vnt + kvh * a.stride_vnh) * 2;
  const int64_t skt = a.stride_knt * 2, svt = a.stride_vnt * 2;

  // pipeline: pages two tiles ahead, K / V one tile ahead (LDS double buffer); one barrier per tile
  DirectPages<D, NW> pages;
  Fp8Tile<D, NW> f8;
  if constexpr (!FP8) {
    if (n_ctx > 0) lookup_direct<D, NW>(pages, kv, lo, hi, wave, lane);
  }
  issue_tile<D, NW, T, FP8>(0, smem, n_ctx, f8, pages, kv, lo, hi, knp, vnp, skt, svt, width, tid, wave, lane);
  if constexpr (FP8) {
    if (n_ctx > 0) store_fp8<D, NW, T>(smem[0][0], smem[0][1], f8, tid);
  } else {
    if (n_ctx > 1) lookup_direct<D, NW>(pages, kv, lo + kTileKeys, hi, wave, lane);
  }

  for (int tile = 0; tile < n_tiles; ++tile) {
    const bool is_new = tile >= n_ctx;
    const int base = is_new ? (tile - n_ctx) * kTileKeys : lo + tile * kTileKeys;  // new tiles: draft row index
    wait_vmem();  // this tile's DMA (issued a tile ago) has landed; the page lookups too
    __syncthreads();  // ... for every wave, and the other buffer is no longer read
    if (tile + 1 < n_tiles) {
      issue_tile<D, NW, T, FP8>(tile + 1, smem, n_ctx, f8, pages, kv, lo, hi, knp, vnp, skt, svt, width, tid, wave,
                                lane);
      if constexpr (!FP8) {
        if (tile + 2 < n_ctx) lookup_direct<D, NW>(pages, kv, lo + (tile + 2) * kTileKeys, hi, wave, lane);
      }
    }
    const char* sKb = smem[tile & 1][0];
    const char* sVb = smem[tile & 1][1];

    if (computes)
      tile_step<D, T>(sKb, sVb, qreg, acc, m, l, scale_log2, is_new, base, hi, width, row_mask, g, l16);
    if constexpr (FP8) {  // the next context tile's dequantised K / V into the other buffer (read after the barrier)
      if (tile + 1 < n_ctx) store_fp8<D, NW, T>(smem[(tile + 1) & 1][0], smem[(tile + 1) & 1][1], f8, tid);
    }
  }

  if (!row_ok) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  if (rq.splits == 1) {
    store_rows<D, T>(static_cast<uint16_t*>(a.out) + (rq.start + t) * a.stride_ot + head * a.stride_oh, acc, inv, g);
  } else {
    const int rows = row_tiles * 16;
    const int64_t part = ((static_cast<int64_t>(b) * a.Hkv + kvh) * max_splits + split) * rows + rho;
    store_partial<D>(a.workspace + part * D, acc, inv, g);
    if (g == 0) {
      float* lse = a.workspace + static_cast<int64_t>(a.num_reqs) * a.Hkv * max_splits * rows * D;
      lse[part] = l > 0.f ? m + log2f(l) : -INFINITY;
    }
  }
}

// vllm/verify_attention.py:115-139 (_verify_merge_kernel) for the requests with more than one split: one thread per
// 4 consecutive d of a row.
template <int D, typename T>
__global__ __launch_bounds__(256) void verify_merge_kernel(const eagle4_attn_args a, int chunk, int row_tiles,
                                                           int max_splits) {
  const int b = blockIdx.z, kvh = blockIdx.y;
  const Req rq = request_info(a, b, chunk);
  if (rq.splits <= 1) return;
  constexpr int TPR = D / 4;
  const int rho = blockIdx.x * (256 / TPR) + threadIdx.x / TPR;
  const int d = 4 * (threadIdx.x % TPR);
  const int G = a.Hq / a.Hkv;
  const int t = rho / G, gq = rho % G;
  const int rows = row_tiles * 16;
  if (rho >= rows || t >= rq.width) return;
  const float* lse = a.workspace + static_cast<int64_t>(a.num_reqs) * a.Hkv * max_splits * rows * D;
  const int64_t part0 = (static_cast<int64_t>(b) * a.Hkv + kvh) * max_splits * rows + rho;
  // The splits in groups of kMergeGroup, every load of a group issued before the first is used (one memory round trip
  // per group, not per split; a group's loads past the last split re-read the first), the same operations in the same
  // order as one split at a time.
  const int ns = rq.splits;
  float mx = -INFINITY;
  for (int s0 = 0; s0 < ns; s0 += kMergeGroup) {
    float l[kMergeGroup];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i) l[i] = lse[part0 + static_cast<int64_t>(s0 + i < ns ? s0 + i : s0) * rows];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i)
      if (s0 + i < ns) mx = fmaxf(mx, l[i]);
  }
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  float wsum = 0.f;
  for (int s0 = 0; s0 < ns; s0 += kMergeGroup) {
    float l[kMergeGroup];
    float4 v[kMergeGroup];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i) {
      const int64_t part = part0 + static_cast<int64_t>(s0 + i < ns ? s0 + i : s0) * rows;
      l[i] = lse[part];
      v[i] = *reinterpret_cast<const float4*>(a.workspace + part * D + d);
    }
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i) {
      if (s0 + i >= ns) break;
      const float w = l[i] == -INFINITY ? 0.f : exp2f(l[i] - mx);
      sum.x += w * v[i].x;
      sum.y += w * v[i].y;
      sum.z += w * v[i].z;
      sum.w += w * v[i].w;
      wsum += w;
    }
  }
  const float inv = 1.0f / wsum;
  uint16_t* op = static_cast<uint16_t*>(a.out) + (rq.start + t) * a.stride_ot + (static_cast<int64_t>(kvh) * G + gq) * a.stride_oh + d;
  uint2 w;
  w.x = static_cast<uint32_t>(T::from_f32(sum.x * inv)) | (static_cast<uint32_t>(T::from_f32(sum.y * inv)) << 16);
  w.y = static_cast<uint32_t>(T::from_f32(sum.z * inv)) | (static_cast<uint32_t>(T::from_f32(sum.w * inv)) << 16);
  *reinterpret_cast<uint2*>(op) = w;
}

struct Plan {
  int chunk, row_tiles, waves, row_groups, max_splits;
};

// 16-row tiles; a workgroup takes up to 8 of them (more rows: more row groups, each reading the KV once).
Plan plan(const eagle4_attn_args& a) {
  Plan p;
  p.chunk = a.chunk > 0 ? a.chunk : (small_attention_job(a) ? kSmallJobChunk : 1024);
  const int G = a.Hq / a.Hkv;
  p.row_tiles = e4::ceil_div(static_cast<int64_t>(G) * a.max_query_len, 16);
  const int need = p.row_tiles < 8 ? p.row_tiles : 8;
  p.waves = need <= 2 ? 2 : (need <= 4 ? 4 : (need <= 6 ? 6 : 8));
  p.row_groups = e4::ceil_div(p.row_tiles, p.waves);
  const int64_t capacity = static_cast<int64_t>(a.max_blocks) * a.page;
  p.max_splits = capacity > 0 ? e4::ceil_div(capacity, p.chunk) : 1;
  return p;
}

// The contract every schedule shares: GQA heads, at most 64 rows per request, int32 page table rows, head dim.
bool shapes_ok(const eagle4_attn_args& a) {
  if (a.Hkv <= 0 || a.Hq % a.Hkv != 0 || a.max_query_len < 1 || a.max_query_len > 64 || a.page < 1) return false;
  if (a.block_table.dtype != EAGLE4_I32 || a.block_table.s1 != 1) return false;
  if (static_cast<int64_t>(a.max_blocks) * a.page >= (int64_t(1) << 31)) return false;  // 32-bit positions
  return a.D == 32 || a.D == 64 || a.D == 128 || a.D == 256;
}

bool covered(const eagle4_attn_args& a) {
  if (!shapes_ok(a)) return false;
  if (a.dtype != EAGLE4_BF16 && a.dtype != EAGLE4_F16) return false;
  if (a.cache_dtype != a.dtype && a.cache_dtype != EAGLE4_FP8_E4M3) return false;
  if (a.cache_dtype == EAGLE4_FP8_E4M3 && (a.k_scale == nullptr || a.v_scale == nullptr)) return false;
  const int chunk = a.chunk > 0 ? a.chunk : (small_attention_job(a) ? kSmallJobChunk : 1024);
  if (chunk % kTileKeys != 0) return false;
  if (static_cast<int64_t>(a.max_blocks) * a.page >= (int64_t(1) << 31)) return false;  // 32-bit positions
  // 16-byte vector accesses along D
  if ((a.stride_qt | a.stride_qh | a.stride_knt | a.stride_knh | a.stride_vnt | a.stride_vnh | a.stride_ot |
       a.stride_oh) % 8 != 0)
    return false;
  if (a.cache_dtype != EAGLE4_FP8_E4M3 &&
      (a.stride_kb | a.stride_ks | a.stride_kh | a.stride_vb | a.stride_vs | a.stride_vh) % 8 != 0)
    return false;
  if (a.cache_dtype == EAGLE4_FP8_E4M3 &&
      (a.stride_kb | a.stride_ks | a.stride_kh | a.stride_vb | a.stride_vs | a.stride_vh) % 8 != 0)
    return false;
  return true;
}

template <int D, int NW, typename T, bool FP8>
int launch(const eagle4_attn_args& a, const Plan& p, hipStream_t s) {
  const dim3 grid(p.max_splits, a.Hkv * p.row_groups, a.num_reqs);
  verify_attention_kernel<D, NW, T, FP8><<<grid, 64 * NW, 0, s>>>(a, p.chunk, p.row_tiles, p.max_splits);
  if (p.max_splits > 1) {
    constexpr int RPB = 256 / (D / 4);
    const dim3 mgrid(e4::ceil_div(p.row_tiles * 16, RPB), a.Hkv, a.num_reqs);
    verify_merge_kernel<D, T><<<mgrid, 256, 0, s>>>(a, p.chunk, p.row_tiles, p.max_splits);
  }
  return E4_LAUNCH_STATUS();
}

template <int D, typename T, bool FP8>
int launch_w(const eagle4_attn_args& a, const Plan& p, hipStream_t s) {
  switch (p.waves) {
    case 2: return launch<D, 2, T, FP8>(a, p, s);
    case 4: return launch<D, 4, T, FP8>(a, p, s);
    case 6: return launch<D, 6, T, FP8>(a, p, s);
    default: return launch<D, 8, T, FP8>(a, p, s);
  }
}

template <int D>
int launch_d(const eagle4_attn_args& a, const Plan& p, hipStream_t s) {
  const bool fp8 = a.cache_dtype == EAGLE4_FP8_E4M3;
  if (a.dtype == EAGLE4_BF16) return fp8 ? launch_w<D, e4::Bf16, true>(a, p, s) : launch_w<D, e4::Bf16, false>(a, p, s);
  return fp8 ? launch_w<D, e4::F16, true>(a, p, s) : launch_w<D, e4::F16, false>(a, p, s);
}

}  // namespace

extern "C" int64_t eagle4_verify_attention_workspace(const eagle4_attn_args* a) {
  if (a->dtype == EAGLE4_F32) return shapes_ok(*a) && f32_covered(*a) ? f32_workspace_bytes(*a) : -1;
  if (!covered(*a)) return -1;
  StreamPlan sp;
  if (stream_covered(*a) && stream_plan(*a, sp)) return stream_workspace_bytes(sp, *a);
  const Plan p = plan(*a);
  if (p.max_splits <= 1) return 0;
  const int64_t parts = static_cast<int64_t>(a->num_reqs) * a->Hkv * p.max_splits * p.row_tiles * 16;
  return parts * (a->D + 1) * static_cast<int64_t>(sizeof(float));
}

// 16-bit rows: up to 1024 requests with the library's split take the streamed schedule (16-bit or fp8 pages), the
// rest the split-context one. fp32 rows over fp32 pages: their own split-context kernel.
extern "C" int eagle4_verify_attention(const eagle4_attn_args* a, void* stream) {
  if (a->num_reqs == 0) return EAGLE4_OK;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->dtype == EAGLE4_F32) return shapes_ok(*a) && f32_covered(*a) ? f32_launch(*a, s) : EAGLE4_NOT_COVERED;
  if (!covered(*a)) return EAGLE4_NOT_COVERED;
  StreamPlan sp;
  if (stream_covered(*a) && stream_plan(*a, sp)) {
    if (a->workspace == nullptr || a->workspace_bytes < stream_workspace_bytes(sp, *a)) return EAGLE4_NOT_COVERED;
    return stream_launch(*a, sp, s);
  }
  const Plan p = plan(*a);
  if (p.max_splits > 1 && (a->workspace == nullptr || a->workspace_bytes < eagle4_verify_attention_workspace(a)))
    return EAGLE4_NOT_COVERED;
  switch (a->D) {
    case 32: return launch_d<32>(*a, p, s);
    case 64: return launch_d<64>(*a, p, s);
    case 128: return launch_d<128>(*a, p, s);
    default: return launch_d<256>(*a, p, s);
  }
}
