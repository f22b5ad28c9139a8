// Tree-verify attention on gfx950: GQA rows over a paged (bf16 / f16 / fp8-e4m3) KV cache plus the round's draft
// rows (vllm/verify_attention.py:29-207, kernels/online_softmax.py:11-24).
//
// Roofline: HBM reads of the KV cache (~94 FLOP/B at batch 64, tree width 16, GQA 6, D 256; the bf16 MFMA ridge is
// ~310 FLOP/B). The design reads every KV byte once:
//
//  * One workgroup per (split of the context, KV head, request): its 4 waves own up to 4 tiles of 32 query rows,
//    where a row is (draft token, query head of the KV head's group), so the G x W rows of a KV head share one read
//    of each K / V tile (the reference's grid is per query head and re-reads every tile G times).
//  * Splits are fixed-size context chunks; a request uses ceil(L / chunk) of them (the grid is sized for the page
//    table's capacity and idle splits exit at once). The last split also takes the draft keys, masked by the rows'
//    ancestor bits. A request with one split writes its output directly; others write fp32 partials with their
//    log2-sum-exp, merged by a second kernel.
//  * 64-key tiles are staged in LDS: K row-major (row pitch D + 8 elements, conflict-free 16-byte reads), V transposed
//    to [d][key] in registers (8x8 16-bit transposes) with an XOR swizzle so both the transposing writes and the
//    MFMA operand reads are conflict-free. fp8 pages are dequantised (x * scale of the (page, KV head)) into the same
//    16-bit tiles as they are staged.
//  * Scores are S^T = K Q^T (v_mfma_f32_32x32x16): a lane then holds one query row's 16 scores per 32 keys, so the
//    online softmax needs one cross-half exchange per row, and P^T is the B operand of O^T = V^T P^T directly in
//    registers. O^T keeps one row per lane, so the rescale by exp2(m_old - m_new) is a per-lane multiply.

#include <type_traits>

#include "common.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTileKeys = 64;

template <typename T>
E4_DEV f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
  if constexpr (T::code == EAGLE4_BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

// Two fp32 values rounded (nearest even) to 16-bit dtype T and packed, low first: one v_cvt_pk_* on gfx950.
template <typename T>
E4_DEV uint32_t pack2(float x, float y) {
  if constexpr (T::code == EAGLE4_BF16) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {static_cast<__bf16>(x), static_cast<__bf16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t v = {static_cast<_Float16>(x), static_cast<_Float16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  }
}

// 8x8 transpose of 16-bit values: in[i] holds d = 0..7 of key i; out[j] holds keys 0..7 of d = j.
E4_DEV void transpose8x8(const uint4 (&in)[8], uint4 (&out)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint4& lo = in[2 * p];
      const uint4& hi = in[2 * p + 1];
      const uint32_t lw = (j >> 1) == 0 ? lo.x : (j >> 1) == 1 ? lo.y : (j >> 1) == 2 ? lo.z : lo.w;
      const uint32_t hw = (j >> 1) == 0 ? hi.x : (j >> 1) == 1 ? hi.y : (j >> 1) == 2 ? hi.z : hi.w;
      w[p] = __builtin_amdgcn_perm(hw, lw, sel);
    }
    out[j] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// 8 fp8-e4m3 values (OCP) times a scale, rounded to 16-bit dtype T, packed.
template <typename T>
E4_DEV uint4 dequant8(uint2 raw, float scale) {
  const auto f0 = __builtin_amdgcn_cvt_pk_f32_fp8(raw.x, false);  // bytes 0, 1
  const auto f1 = __builtin_amdgcn_cvt_pk_f32_fp8(raw.x, true);   // bytes 2, 3
  const auto f2 = __builtin_amdgcn_cvt_pk_f32_fp8(raw.y, false);
  const auto f3 = __builtin_amdgcn_cvt_pk_f32_fp8(raw.y, true);
  auto pack = [scale](float x, float y) { return pack2<T>(x * scale, y * scale); };
  return make_uint4(pack(f0[0], f0[1]), pack(f1[0], f1[1]), pack(f2[0], f2[1]), pack(f3[0], f3[1]));
}

// The 8 keys of V-transpose group g (0..7) of a 64-key tile, in the order of the PV operand (key' = 8g + i).
E4_DEV int group_key(int g, int i) { return 32 * (g >> 2) + 16 * ((g >> 1) & 1) + 8 * (i >> 2) + 4 * (g & 1) + (i & 3); }

// Byte offset of the 16-byte chunk (row d, logical chunk g) of the swizzled V^T tile (rows of 64 keys = 128 bytes).
E4_DEV int vt_offset(int d, int g) { return d * 128 + 16 * (g ^ ((d + (d >> 3)) & 7)); }

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

// One thread's share of a 64-key K / V tile, loaded ahead into registers (raw cache bytes; fp8 with its scales) and
// written to LDS one tile later, so the next tile's HBM reads overlap this tile's MFMAs.
template <int D, bool FP8>
struct TileRegs {
  using Raw = typename std::conditional<FP8, uint2, uint4>::type;
  static constexpr int NK = D / 32;  // K (key, 8-element chunk) pairs per thread: 64 * D / 8 / 256
  Raw k[NK];
  Raw v[8];
  float ks[NK], vs[8];
};

template <int D, typename T, bool FP8>
E4_DEV void load_tile(TileRegs<D, FP8>& r, const KvAddr& kv, int base, int hi, int tid) {
  using Raw = typename TileRegs<D, FP8>::Raw;
  constexpr int KCH = D / 8;
  constexpr int EB = FP8 ? 1 : 2;  // bytes per element
  const Raw zero{};
#pragma unroll
  for (int i = 0; i < TileRegs<D, FP8>::NK; ++i) {
    const int q = tid + 256 * i;
    const int key = q / KCH, dc = q % KCH;
    r.k[i] = zero;
    r.ks[i] = 1.f;
    const int pos = base + key;
    if (pos < hi) {
      int bi, sl;
      page_of(kv, pos, bi, sl);
      const int64_t blk = kv.bt[bi];
      r.k[i] = *reinterpret_cast<const Raw*>(kv.kbase + blk * kv.kb + sl * kv.ks + 8 * EB * dc);
      if constexpr (FP8) r.ks[i] = kv.kscale[blk * kv.ksb];
    }
  }
  if (tid < 8 * KCH) {
    const int g = tid / KCH, dc = tid % KCH;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      r.v[i] = zero;
      r.vs[i] = 1.f;
      const int pos = base + group_key(g, i);
      if (pos < hi) {
        int bi, sl;
        page_of(kv, pos, bi, sl);
        const int64_t blk = kv.bt[bi];
        r.v[i] = *reinterpret_cast<const Raw*>(kv.vbase + blk * kv.vb + sl * kv.vs + 8 * EB * dc);
        if constexpr (FP8) r.vs[i] = kv.vscale[blk * kv.vsb];
      }
    }
  }
}

// The draft keys / values (16-bit even with an fp8 cache) go straight into 16-bit registers.
template <int D>
E4_DEV void load_new_16(uint4 (&k)[D / 32], uint4 (&v)[8], const char* kn, const char* vn, int64_t skt, int64_t svt,
                        int width, int tid) {
  constexpr int KCH = D / 8;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const int q = tid + 256 * i;
    const int key = q / KCH, dc = q % KCH;
    k[i] = key < width ? *reinterpret_cast<const uint4*>(kn + key * skt + 16 * dc) : make_uint4(0, 0, 0, 0);
  }
  if (tid < 8 * KCH) {
    const int g = tid / KCH, dc = tid % KCH;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = group_key(g, i);
      v[i] = key < width ? *reinterpret_cast<const uint4*>(vn + key * svt + 16 * dc) : make_uint4(0, 0, 0, 0);
    }
  }
}

template <int D>
E4_DEV void store_tile_16(uint16_t* sK, uint16_t* sVt, const uint4 (&k)[D / 32], const uint4 (&v)[8], int tid) {
  constexpr int KCH = D / 8, KP = D + 8;
#pragma unroll
  for (int i = 0; i < D / 32; ++i) {
    const int q = tid + 256 * i;
    *reinterpret_cast<uint4*>(&sK[(q / KCH) * KP + 8 * (q % KCH)]) = k[i];
  }
  if (tid < 8 * KCH) {
    const int g = tid / KCH, dc = tid % KCH;
    uint4 out[8];
    transpose8x8(v, out);
    char* vt = reinterpret_cast<char*>(sVt);
#pragma unroll
    for (int j = 0; j < 8; ++j) *reinterpret_cast<uint4*>(vt + vt_offset(8 * dc + j, g)) = out[j];
  }
}

template <int D, typename T, bool FP8>
E4_DEV void store_tile(uint16_t* sK, uint16_t* sVt, const TileRegs<D, FP8>& r, int tid) {
  if constexpr (FP8) {
    uint4 k[D / 32], v[8];
#pragma unroll
    for (int i = 0; i < D / 32; ++i) k[i] = dequant8<T>(r.k[i], r.ks[i]);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = dequant8<T>(r.v[i], r.vs[i]);
    store_tile_16<D>(sK, sVt, k, v, tid);
  } else {
    store_tile_16<D>(sK, sVt, r.k, r.v, tid);
  }
}

template <int D, typename T, bool FP8>
__global__ __launch_bounds__(256, 1) void verify_attention_kernel(const eagle4_attn_args a, int chunk, int row_tiles,
                                                                  int max_splits) {
  static_assert(D % 32 == 0 && D >= 32 && D <= 256, "head dim");
  constexpr int KP = D + 8;  // K tile row pitch (elements)
  // D = 256: the Q operands of the 4 waves live in LDS (rows of D + 8 elements) to leave registers to O^T and the
  // prefetched tile; smaller heads keep them in registers.
  constexpr bool kQInLds = D == 256;
  __shared__ __attribute__((aligned(16))) uint16_t sK[kTileKeys * KP];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[D * kTileKeys];
  __shared__ __attribute__((aligned(16))) uint16_t sQ[kQInLds ? 4 * 32 * KP : 8];

  const int split = blockIdx.x;
  const int G = a.Hq / a.Hkv;
  const int kvh = blockIdx.y % a.Hkv;
  const int rgroup = blockIdx.y / a.Hkv;
  const int b = blockIdx.z;
  const Req rq = request_info(a, b, chunk);
  if (split >= rq.splits || rq.width <= 0) return;

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = lane >> 5, l32 = lane & 31;
  const int rt = rgroup * 4 + wave;
  const bool computes = rt < row_tiles;
  const int rho = rt * 32 + l32;  // this lane's query row
  const int t = rho / G, gq = rho % G;
  const bool row_ok = computes && t < rq.width && t < a.max_query_len;
  const int64_t head = static_cast<int64_t>(kvh) * G + gq;

  // Q of the lane's row: d = 16 s + 8 h + (0..7) for s < D / 16
  constexpr int QN = kQInLds ? 1 : D / 16;
  uint4 qreg[QN];
  const uint16_t* sQrow = &sQ[kQInLds ? (wave * 32 + l32) * KP + 8 * h : 0];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + (rq.start + t) * a.stride_qt + head * a.stride_qh + 8 * h;
#pragma unroll
    for (int s = 0; s < D / 16; ++s) {
      const uint4 qv = row_ok ? *reinterpret_cast<const uint4*>(qp + 16 * s) : make_uint4(0, 0, 0, 0);
      if constexpr (kQInLds)
        *reinterpret_cast<uint4*>(const_cast<uint16_t*>(sQrow) + 16 * s) = qv;
      else
        qreg[s] = qv;
    }
  }
  int64_t row_mask = 0;
  if (row_ok) row_mask = a.masks[b * a.stride_mask + t];

  f32x16_t acc[D / 32];
#pragma unroll
  for (int i = 0; i < D / 32; ++i) acc[i] = f32x16_t{};
  float m = -INFINITY, l = 0.f;
  const float scale_log2 = a.scale * 1.4426950408889634f;

  const int64_t lo = static_cast<int64_t>(split) * chunk;  // context positions stay below 2^31
  const int64_t hi = lo + chunk < rq.context ? lo + chunk : rq.context;
  const bool has_new = split == rq.splits - 1;
  const int n_ctx_tiles = hi > lo ? static_cast<int>((hi - lo + kTileKeys - 1) / kTileKeys) : 0;
  const int n_tiles = n_ctx_tiles + (has_new ? 1 : 0);

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
  const int ilo = static_cast<int>(lo), ihi = static_cast<int>(hi);
  TileRegs<D, FP8> pre;
  if (n_ctx_tiles > 0) load_tile<D, T, FP8>(pre, kv, ilo, ihi, tid);
  for (int tile = 0; tile < n_tiles; ++tile) {
    const bool is_new = tile == n_ctx_tiles;
    const int64_t base = lo + static_cast<int64_t>(tile) * kTileKeys;
    // ---- stage this tile: K row-major, V transposed (the previous tile's MFMAs are done: barrier) -------------------
    __syncthreads();
    if (is_new) {
      uint4 kn[D / 32], vn[8];
      const char* knp = static_cast<const char*>(a.k_new) + (rq.start * a.stride_knt + kvh * a.stride_knh) * 2;
      const char* vnp = static_cast<const char*>(a.v_new) + (rq.start * a.stride_vnt + kvh * a.stride_vnh) * 2;
      load_new_16<D>(kn, vn, knp, vnp, a.stride_knt * 2, a.stride_vnt * 2, static_cast<int>(rq.width), tid);
      store_tile_16<D>(sK, sVt, kn, vn, tid);
    } else {
      store_tile<D, T, FP8>(sK, sVt, pre, tid);
    }
    __syncthreads();
    if (tile + 1 < n_ctx_tiles) load_tile<D, T, FP8>(pre, kv, static_cast<int>(base) + kTileKeys, ihi, tid);

    if (computes) {
      // ---- S^T = K Q^T for keys 0..31 and 32..63 ----------------------------------------------------------------
      f32x16_t s[2] = {f32x16_t{}, f32x16_t{}};
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const uint16_t* kr = &sK[(32 * sb + l32) * KP + 8 * h];
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          uint4 qv;
          if constexpr (kQInLds)
            qv = *reinterpret_cast<const uint4*>(sQrow + 16 * c);
          else
            qv = qreg[c];
          s[sb] = mfma32<T>(*reinterpret_cast<const uint4*>(kr + 16 * c), qv, s[sb]);
          // keep the operand reads next to their MFMAs (hoisting them all costs a register per byte of the tile)
          if ((c & 3) == 3) __builtin_amdgcn_sched_barrier(0);
        }
      }
      // ---- mask, online softmax (log2 domain) -------------------------------------------------------------------
      float tmax = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = 32 * sb + 8 * (j >> 2) + 4 * h + (j & 3);
          bool ok;
          if (is_new)
            ok = key < rq.width && ((row_mask >> key) & 1);
          else
            ok = static_cast<int>(base) + key < ihi;
          const float v = ok ? s[sb][j] * scale_log2 : -INFINITY;
          s[sb][j] = v;
          tmax = fmaxf(tmax, v);
        }
      }
      tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
      const float m_new = fmaxf(m, tmax);
      const float safe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m - safe);
      float psum = 0.f;
      uint4 pb[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const float p0 = exp2f(s[c >> 1][8 * (c & 1) + 2 * p] - safe);
          const float p1 = exp2f(s[c >> 1][8 * (c & 1) + 2 * p + 1] - safe);
          psum += p0 + p1;
          w[p] = pack2<T>(p0, p1);
        }
        pb[c] = make_uint4(w[0], w[1], w[2], w[3]);
      }
      psum += __shfl_xor(psum, 32, 64);
      l = l * alpha + psum;
      m = m_new;
      // ---- O^T = O^T * alpha + V^T P^T -------------------------------------------------------------------------
      const char* vt = reinterpret_cast<const char*>(sVt);
#pragma unroll
      for (int dt = 0; dt < D / 32; ++dt) {
        acc[dt] *= alpha;
        const int d = 32 * dt + l32;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          acc[dt] = mfma32<T>(*reinterpret_cast<const uint4*>(vt + vt_offset(d, 2 * c + h)), pb[c], acc[dt]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  if (!row_ok) return;
  const float inv = l > 0.f ? 1.0f / l : 0.f;
  if (rq.splits == 1) {
    uint16_t* op = static_cast<uint16_t*>(a.out) + (rq.start + t) * a.stride_ot + head * a.stride_oh;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * h;
        uint2 w;
        w.x = static_cast<uint32_t>(T::from_f32(acc[dt][4 * g4] * inv)) |
              (static_cast<uint32_t>(T::from_f32(acc[dt][4 * g4 + 1] * inv)) << 16);
        w.y = static_cast<uint32_t>(T::from_f32(acc[dt][4 * g4 + 2] * inv)) |
              (static_cast<uint32_t>(T::from_f32(acc[dt][4 * g4 + 3] * inv)) << 16);
        *reinterpret_cast<uint2*>(op + d) = w;
      }
  } else {
    const int rows = row_tiles * 32;
    const int64_t part = ((static_cast<int64_t>(b) * a.Hkv + kvh) * max_splits + split) * rows + rho;
    float* pp = a.workspace + part * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d = 32 * dt + 8 * g4 + 4 * h;
        *reinterpret_cast<float4*>(pp + d) = make_float4(acc[dt][4 * g4] * inv, acc[dt][4 * g4 + 1] * inv,
                                                         acc[dt][4 * g4 + 2] * inv, acc[dt][4 * g4 + 3] * inv);
      }
    if (h == 0) {
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
  const int rows = row_tiles * 32;
  if (rho >= rows || t >= rq.width) return;
  const float* lse = a.workspace + static_cast<int64_t>(a.num_reqs) * a.Hkv * max_splits * rows * D;
  const int64_t part0 = (static_cast<int64_t>(b) * a.Hkv + kvh) * max_splits * rows + rho;
  float mx = -INFINITY;
  for (int s = 0; s < rq.splits; ++s) mx = fmaxf(mx, lse[part0 + static_cast<int64_t>(s) * rows]);
  float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
  float wsum = 0.f;
  for (int s = 0; s < rq.splits; ++s) {
    const int64_t part = part0 + static_cast<int64_t>(s) * rows;
    const float ls = lse[part];
    const float w = ls == -INFINITY ? 0.f : exp2f(ls - mx);
    const float4 v = *reinterpret_cast<const float4*>(a.workspace + part * D + d);
    sum.x += w * v.x;
    sum.y += w * v.y;
    sum.z += w * v.z;
    sum.w += w * v.w;
    wsum += w;
  }
  const float inv = 1.0f / wsum;
  uint16_t* op = static_cast<uint16_t*>(a.out) + (rq.start + t) * a.stride_ot + (static_cast<int64_t>(kvh) * G + gq) * a.stride_oh + d;
  uint2 w;
  w.x = static_cast<uint32_t>(T::from_f32(sum.x * inv)) | (static_cast<uint32_t>(T::from_f32(sum.y * inv)) << 16);
  w.y = static_cast<uint32_t>(T::from_f32(sum.z * inv)) | (static_cast<uint32_t>(T::from_f32(sum.w * inv)) << 16);
  *reinterpret_cast<uint2*>(op) = w;
}

struct Plan {
  int chunk, row_tiles, row_groups, max_splits;
};

Plan plan(const eagle4_attn_args& a) {
  Plan p;
  p.chunk = a.chunk > 0 ? a.chunk : 1024;
  const int G = a.Hq / a.Hkv;
  p.row_tiles = e4::ceil_div(static_cast<int64_t>(G) * a.max_query_len, 32);
  p.row_groups = e4::ceil_div(p.row_tiles, 4);
  const int64_t capacity = static_cast<int64_t>(a.max_blocks) * a.page;
  p.max_splits = capacity > 0 ? e4::ceil_div(capacity, p.chunk) : 1;
  return p;
}

bool covered(const eagle4_attn_args& a) {
  if (a.Hkv <= 0 || a.Hq % a.Hkv != 0 || a.max_query_len < 1 || a.max_query_len > 64 || a.page < 1) return false;
  if (a.block_table.dtype != EAGLE4_I32 || a.block_table.s1 != 1) return false;
  if (a.D != 32 && a.D != 64 && a.D != 128 && a.D != 256) return false;
  if (a.dtype != EAGLE4_BF16 && a.dtype != EAGLE4_F16) return false;
  if (a.cache_dtype != a.dtype && a.cache_dtype != EAGLE4_FP8_E4M3) return false;
  if (a.cache_dtype == EAGLE4_FP8_E4M3 && (a.k_scale == nullptr || a.v_scale == nullptr)) return false;
  const int chunk = a.chunk > 0 ? a.chunk : 1024;
  if (chunk % kTileKeys != 0) return false;
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

template <int D, typename T, bool FP8>
int launch(const eagle4_attn_args& a, const Plan& p, hipStream_t s) {
  const dim3 grid(p.max_splits, a.Hkv * p.row_groups, a.num_reqs);
  verify_attention_kernel<D, T, FP8><<<grid, 256, 0, s>>>(a, p.chunk, p.row_tiles, p.max_splits);
  if (p.max_splits > 1) {
    constexpr int RPB = 256 / (D / 4);
    const dim3 mgrid(e4::ceil_div(p.row_tiles * 32, RPB), a.Hkv, a.num_reqs);
    verify_merge_kernel<D, T><<<mgrid, 256, 0, s>>>(a, p.chunk, p.row_tiles, p.max_splits);
  }
  return E4_LAUNCH_STATUS();
}

template <int D>
int launch_d(const eagle4_attn_args& a, const Plan& p, hipStream_t s) {
  const bool fp8 = a.cache_dtype == EAGLE4_FP8_E4M3;
  if (a.dtype == EAGLE4_BF16) return fp8 ? launch<D, e4::Bf16, true>(a, p, s) : launch<D, e4::Bf16, false>(a, p, s);
  return fp8 ? launch<D, e4::F16, true>(a, p, s) : launch<D, e4::F16, false>(a, p, s);
}

}  // namespace

extern "C" int64_t eagle4_verify_attention_workspace(const eagle4_attn_args* a) {
  if (!covered(*a)) return -1;
  const Plan p = plan(*a);
  if (p.max_splits <= 1) return 0;
  const int64_t parts = static_cast<int64_t>(a->num_reqs) * a->Hkv * p.max_splits * p.row_tiles * 32;
  return parts * (a->D + 1) * static_cast<int64_t>(sizeof(float));
}

extern "C" int eagle4_verify_attention(const eagle4_attn_args* a, void* stream) {
  if (a->num_reqs == 0) return EAGLE4_OK;
  if (!covered(*a)) return EAGLE4_NOT_COVERED;
  const Plan p = plan(*a);
  if (p.max_splits > 1 && (a->workspace == nullptr || a->workspace_bytes < eagle4_verify_attention_workspace(a)))
    return EAGLE4_NOT_COVERED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->D) {
    case 32: return launch_d<32>(*a, p, s);
    case 64: return launch_d<64>(*a, p, s);
    case 128: return launch_d<128>(*a, p, s);
    default: return launch_d<256>(*a, p, s);
  }
}
