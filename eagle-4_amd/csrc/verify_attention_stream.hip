// Tree-verify attention over paged KV caches (16-bit, or fp8-e4m3 with per-(page, KV head) scales), streamed
// (vllm/verify_attention.py:29-207 computes the same rows; this is its schedule for gfx950).
//
// The work is the sequence of 32-key tiles of every segment — (request, KV head, row group), context tiles then
// draft tiles — in request order. A persistent grid of one workgroup per resident slot takes equal contiguous shares
// of that sequence, so every CU streams the same number of KV bytes whatever the context lengths are, and no
// workgroup drains its pipeline between segments. A segment that lies inside one share is normalised and written
// directly; one cut by share boundaries leaves fp32 partials (with their log2-sum-exp), at most two per share (its
// first and its last piece), in slots numbered by the share, so the workspace is bounded by the grid whatever the
// batch; a second kernel merges them.
//
// A workgroup is C consumer waves, each owning 16 query rows (a row is a (draft token, query head of the KV head's
// group) pair, so one read of a K / V tile serves all G W rows), and two producer waves. The producers run the page
// lookups and the K / V loads of a kStages-deep LDS ring; iteration x computes tile x while tiles x + 1 .. x + S - 1
// are in flight (two producers: a wave holds at most 63 loads in flight, fewer than S - 1 tiles' 1 KB loads). Loads
// and lookups are LDS DMA (global_load_lds) issued from inline assembly: the compiler cannot see them, so it does not
// drain the load counter before the consumers' LDS reads; each producer waits explicitly — vmcnt(n) with n the loads
// it issued after the ones tile x needs, exact because vector loads retire in issue order — and a barrier per tile
// hands the tile over. When a load instruction's rows share one page (page sizes dividing 32
// or multiples of 32), its address is a scalar page base plus a per-lane constant.
//
// Roofline: HBM reads of K and V (2 D bytes per key per KV head and row group); the MFMA work per tile (G W rows
// against 32 keys) is a fraction of the bf16 ridge, so the design target is bytes in flight.

#include "attention_tile.h"

#pragma clang diagnostic ignored "-Winline-asm"  // the direct loads set M0; no compiler-generated code here uses M0

namespace e4attn {

constexpr int kStages = 4;            // power of two
constexpr int kProducers = 2;
constexpr int kMinTilesPerGroup = 8;  // small jobs use fewer, longer shares
constexpr int kAheadTiles = 4;        // tiles before a segment's end that its successor's rows are loaded (16-bit pages)

namespace {

E4_DEV int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }

E4_DEV uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// 64 lanes x 16 bytes from per-lane global addresses into LDS [lds, lds + 1024), lane p at lds + 16 p. The K / V
// stream is read once, with the nontemporal policy: its lines do not displace what the last-level cache holds, so
// the dirty lines a previous kernel left there (the state commit's stores before the next step's attention) are not
// written back in the middle of the stream (batch-64 step 0.824 -> 0.774 ms: the attention 311 -> 264 us, the commit
// 58 -> 77 us, which now finds those lines still to be written back).
E4_DEV void dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(lds) : "memory", "m0");
}

// The same from a scalar base plus per-lane 32-bit offsets.
E4_DEV void dma16s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}

// 64 lanes x 4 bytes into LDS [lds, lds + 256).
E4_DEV void dma4(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

template <int N>
E4_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Position in the tile sequence: request b, segment k of the request (KV head k / RG, row group k % RG), tile j of
// the segment; with the request's tile counts, context length, query start and draft width (keys, at most 64).
struct Cursor {
  int b, k, j;
  int tiles, n_ctx, ctx, qs, width;
};

// CK: keys of a context tile (32 for 16-bit pages, 64 for fp8); draft tiles hold 32 keys.
template <int CK>
E4_DEV void cur_load(Cursor& c, const int* s_qsl, const int* s_ctx, int B) {
  if (c.b >= B) {  // past the last request (a look-ahead cursor): an empty draft tile
    c.tiles = 1;
    c.n_ctx = 0;
    c.ctx = 0;
    c.qs = 0;
    c.width = 1;
    return;
  }
  c.qs = uni(s_qsl[c.b]);
  const int w = uni(s_qsl[c.b + 1]) - c.qs;
  c.width = w < 64 ? w : 64;
  c.ctx = uni(s_ctx[c.b]);
  c.n_ctx = c.width > 0 ? (c.ctx + CK - 1) / CK : 0;
  c.tiles = c.width > 0 ? c.n_ctx + (c.width + kTileKeys - 1) / kTileKeys : 0;
}

template <int CK>
E4_DEV void cur_next(Cursor& c, const int* s_qsl, const int* s_ctx, int B, int HR) {
  if (++c.j < c.tiles) return;
  c.j = 0;
  if (++c.k < HR) return;
  c.k = 0;
  do {
    ++c.b;
    cur_load<CK>(c, s_qsl, s_ctx, B);
  } while (c.tiles == 0);
}

template <int CK>
E4_DEV int tiles_of(const int* s_qsl, const int* s_ctx, int b) {
  const int w = s_qsl[b + 1] - s_qsl[b];
  if (w <= 0) return 0;
  const int wk = w < 64 ? w : 64;
  return (s_ctx[b] + CK - 1) / CK + (wk + kTileKeys - 1) / kTileKeys;
}

E4_DEV int64_t active_groups(int64_t tiles_all, int nwg) {
  const int64_t n = (tiles_all + kMinTilesPerGroup - 1) / kMinTilesPerGroup;
  return n < nwg ? n : nwg;
}

E4_DEV int page_div(int pos, int page, int shift) {
  return shift >= 0 ? pos >> shift : static_cast<int>(static_cast<uint32_t>(pos) / static_cast<uint32_t>(page));
}

// 16 bytes from LDS byte address `addr`; the transposing 8-byte read (ds_read_b64_tr_b16) at `addr`.
E4_DEV u32x4_t lds_load16(uint32_t addr) {
  return *(const __attribute__((address_space(3))) u32x4_t*)static_cast<uintptr_t>(addr);
}
E4_DEV v4i16 lds_tr16(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16*)static_cast<uintptr_t>(addr));
}

// Per-lane LDS offsets of a consumer's operand reads within a stage. The swizzles XOR only the chunk-index bits that
// Tile::KB / Tile::VB count, and rows 16 apart share a swizzle, so each read is a base plus an immediate: K chunk
// 4 c + g of key row 16 kt + l16 sits at kb[c % KB] + 16 ROWB kt + 64 KB (c / KB); the transposing V reads of d-tile dt
// (keys 16 h + 4 g + j, h = 0, 1, j = l16 / 4) at vb[dt % VB] + 16 ROWB h + 32 VB (dt / VB).
struct OperandOffsets {
  uint32_t kb[4];
  uint32_t vb[8];
};

template <int D>
E4_DEV OperandOffsets operand_offsets(int g, int l16) {
  using TL = Tile<D>;
  static_assert(TL::kswz(16) == TL::kswz(0) && TL::vswz(16) == TL::vswz(0), "rows 16 apart share a swizzle");
  OperandOffsets o = {};
#pragma unroll
  for (int e = 0; e < TL::KB; ++e) o.kb[e] = l16 * TL::ROWB + 16 * ((4 * e + g) ^ TL::kswz(l16));
  const int j = l16 >> 2, s4 = l16 & 3;
  const int key = 4 * g + j;
#pragma unroll
  for (int v = 0; v < TL::VB; ++v)
    o.vb[v] = TL::BYTES + key * TL::ROWB + 16 * ((2 * v + (s4 >> 1)) ^ TL::vswz(key)) + 8 * (s4 & 1);
  return o;
}

// The same for fp8 context tiles (Tile8): K chunk 2 c + g / 2 (half g & 1) of key row 16 kt + l16 at
// kb[kt][c & 3] + 128 (c >> 2); the transposing V read of d-tile dt by lane l16 — key row 16 (k / 4) + 4 g + k % 4 with
// k = l16 / 2, half l16 & 1 — at vb[dt & 7] + 128 (dt >> 3). ds_read_b64_tr_b8 hands lane j of a 16-lane group byte
// j % 8 of the reads of lanes 2 k + j / 8, k = 0 .. 7: lane l16 then holds d = 16 dt + l16 of keys
// 16 (k / 4) + 4 g + k % 4, the key order of P^T's operand.
struct OperandOffsets8 {
  uint32_t kb[2][4];
  uint32_t vb[8];
};

template <int D>
E4_DEV OperandOffsets8 operand_offsets8(int g, int l16) {
  using T8 = Tile8<D>;
  OperandOffsets8 o;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int key = 16 * kt + l16;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o.kb[kt][e] = key * T8::ROWB + 16 * ((2 * e + (g >> 1)) ^ T8::kswz(key)) + 8 * (g & 1);
  }
  const int k = l16 >> 1;
  const int key = 16 * (k >> 2) + 4 * g + (k & 3);
#pragma unroll
  for (int e = 0; e < 8; ++e) o.vb[e] = key * T8::ROWB + 16 * (e ^ T8::vswz(key)) + 8 * (l16 & 1);
  return o;
}

E4_DEV uint2 lds_load8(uint32_t addr) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = *(const __attribute__((address_space(3))) u32x2*)static_cast<uintptr_t>(addr);
  return make_uint2(v.x, v.y);
}
E4_DEV uint2 lds_tr8(uint32_t addr) {
  typedef int v2i32 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(
      uint2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i32*)static_cast<uintptr_t>(addr)));
}

// Consumer step: one 32-key tile for a wave's 16 rows (lane l16 of each 16-lane group owns row l16; g = lane / 16).
//   S^T = K Q^T on v_mfma_f32_16x16x32 (s[kt][i]: key 16 kt + 4 g + i of the lane's row); scores outside `vis`
//   (bit k: key k of the tile is visible to the row) are -inf. Softmax in the log2 domain against a per-row reference
//   mref that is raised only when a score exceeds it by more than kSlack (then O^T and the lane's partial sum are
//   rescaled): probabilities stay below 2^kSlack and the common step has no cross-lane traffic. O^T += V^T P^T with
//   P^T straight from registers as the B operand and V^T from transposing LDS reads. `stage` is the LDS byte address
//   of the tile's K (V follows it).
// The reference's online-softmax step is kernels/online_softmax.py:11-24, over vllm/verify_attention.py:62-112's
// masked scores; raising the reference lazily changes only fp32 rounding.
template <int D, typename T>
E4_DEV void consume_tile(uint32_t stage, const OperandOffsets& off, const u32x4_t (&q)[D / 32], f32x4_t (&acc)[D / 16],
                         float& mref, float& lsum, float scale_log2, uint32_t vis, bool full, int g) {
  constexpr float kSlack = 16.0f;
  // operands are read in groups (K: KG chunks per key row, V: VG d-tiles), a compiler fence after each group: at
  // most two groups are in registers at once (one being multiplied, the next arriving)
  constexpr int KG = 4, VG = 4;
  using TL = Tile<D>;
  constexpr int KB = TL::KB, VB = TL::VB;
  uint32_t kb[KB];
#pragma unroll
  for (int e = 0; e < KB; ++e) kb[e] = stage + off.kb[e];
  f32x4_t s[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int c0 = 0; c0 < D / 32; c0 += KG) {
    u32x4_t kop[2][KG];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < KG && c0 + c < D / 32; ++c) {
        const int cc = c0 + c;
        kop[kt][c] = lds_load16(kb[cc % KB] + 16 * TL::ROWB * kt + 64 * KB * (cc / KB));
      }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int c = 0; c < KG && c0 + c < D / 32; ++c)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) s[kt] = mfma16<T>(kop[kt][c], q[c0 + c], s[kt]);
  }
  // the V reads' bases for this stage (at D 256 opaque to the compiler, so that 32 VB (dt / VB) stays the reads'
  // offset field)
  uint32_t vb[VB];
#pragma unroll
  for (int v = 0; v < VB; ++v) {
    vb[v] = off.vb[v];
    if constexpr (D == 256) {
      vb[v] += stage;
      asm volatile("" : "+v"(vb[v]));
    }
  }
  const uint32_t vst = D == 256 ? 0u : stage;
  auto read_v = [&](int dt) {
    const uint32_t o = 32 * VB * (dt / VB);
    const v4i16 lo4 = lds_tr16(vst + vb[dt % VB] + o);
    const v4i16 hi4 = lds_tr16(vst + vb[dt % VB] + 16 * TL::ROWB + o);
    return __builtin_shufflevector(__builtin_bit_cast(u32x2_t, lo4), __builtin_bit_cast(u32x2_t, hi4), 0, 1, 2, 3);
  };
  u32x4_t vop[VG];
#pragma unroll
  for (int i = 0; i < VG && i < D / 16; ++i) vop[i] = read_v(i);  // the first group lands while the softmax runs
  asm volatile("" ::: "memory");

  // scaled scores; a tile whose keys are all visible (`full`, wave-uniform) skips the mask
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[kt][i] *= scale_log2;
  if (!full) {
    asm volatile("");  // a branch, not selects: the common full tile runs none of this
    const uint32_t vv = vis >> (4 * g);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[kt][i] = ((vv >> (16 * kt + i)) & 1u) ? s[kt][i] : -INFINITY;
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[kt][i]);
  if (__any(tmax > mref + kSlack)) {  // rare: a new reference for every row of the wave (max over the row's lanes)
    float rm = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    rm = fmaxf(rm, __shfl_xor(rm, 32, 64));
    const float m_new = fmaxf(mref, rm);
    const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mref - m_new);
    mref = m_new;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] *= alpha;
  }
  const float ref = mref == -INFINITY ? 0.f : mref;
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {  // element i of P^T's operand is key 16 (i / 4) + 4 g + i % 4
    const float p0 = __builtin_amdgcn_exp2f(s[p >> 1][2 * (p & 1)] - ref);
    const float p1 = __builtin_amdgcn_exp2f(s[p >> 1][2 * (p & 1) + 1] - ref);
    lsum += p0 + p1;
    w[p] = pack2<T>(p0, p1);
  }
  const u32x4_t pb = {w[0], w[1], w[2], w[3]};
#pragma unroll
  for (int d0 = 0; d0 < D / 16; d0 += VG) {
    u32x4_t nxt[VG];
    if (d0 + VG < D / 16) {
#pragma unroll
      for (int i = 0; i < VG; ++i) nxt[i] = read_v(d0 + VG + i);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < VG && d0 + i < D / 16; ++i) acc[d0 + i] = mfma16<T>(vop[i], pb, acc[d0 + i]);
    if (d0 + VG < D / 16) {
#pragma unroll
      for (int i = 0; i < VG; ++i) vop[i] = nxt[i];
    }
  }
}

// The same step in three phases, for the pipelined consumer loop (16-bit pages): S^T of tile x, then O^T += V^T P^T of
// tile x - 1 (its P^T kept from the iteration before), then tile x's softmax. The PV products do not depend on tile
// x's scores, so they run on the matrix core while the softmax runs on the VALU. Same arithmetic, in the same order per
// accumulator, as consume_tile.
template <int D, typename T>
E4_DEV void qk_phase(uint32_t stage, const OperandOffsets& off, const u32x4_t (&q)[D / 32], f32x4_t (&s)[2]) {
  constexpr int KG = 4;
  using TL = Tile<D>;
  constexpr int KB = TL::KB;
  uint32_t kb[KB];
#pragma unroll
  for (int e = 0; e < KB; ++e) kb[e] = stage + off.kb[e];
  s[0] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  s[1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c0 = 0; c0 < D / 32; c0 += KG) {
    u32x4_t kop[2][KG];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int c = 0; c < KG && c0 + c < D / 32; ++c) {
        const int cc = c0 + c;
        kop[kt][c] = lds_load16(kb[cc % KB] + 16 * TL::ROWB * kt + 64 * KB * (cc / KB));
      }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int c = 0; c < KG && c0 + c < D / 32; ++c)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) s[kt] = mfma16<T>(kop[kt][c], q[c0 + c], s[kt]);
  }
}

template <int D, typename T>
E4_DEV void pv_phase(uint32_t stage, const OperandOffsets& off, const u32x4_t& pb, f32x4_t (&acc)[D / 16]) {
  constexpr int VG = 4;
  using TL = Tile<D>;
  constexpr int VB = TL::VB;
  uint32_t vb[VB];
#pragma unroll
  for (int v = 0; v < VB; ++v) {
    vb[v] = off.vb[v];
    if constexpr (D == 256) {
      vb[v] += stage;
      asm volatile("" : "+v"(vb[v]));
    }
  }
  const uint32_t vst = D == 256 ? 0u : stage;
  auto read_v = [&](int dt) {
    const uint32_t o = 32 * VB * (dt / VB);
    const v4i16 lo4 = lds_tr16(vst + vb[dt % VB] + o);
    const v4i16 hi4 = lds_tr16(vst + vb[dt % VB] + 16 * TL::ROWB + o);
    return __builtin_shufflevector(__builtin_bit_cast(u32x2_t, lo4), __builtin_bit_cast(u32x2_t, hi4), 0, 1, 2, 3);
  };
  u32x4_t vop[VG];
#pragma unroll
  for (int i = 0; i < VG && i < D / 16; ++i) vop[i] = read_v(i);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int d0 = 0; d0 < D / 16; d0 += VG) {
    u32x4_t nxt[VG];
    if (d0 + VG < D / 16) {
#pragma unroll
      for (int i = 0; i < VG; ++i) nxt[i] = read_v(d0 + VG + i);
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < VG && d0 + i < D / 16; ++i) acc[d0 + i] = mfma16<T>(vop[i], pb, acc[d0 + i]);
    if (d0 + VG < D / 16) {
#pragma unroll
      for (int i = 0; i < VG; ++i) vop[i] = nxt[i];
    }
  }
}

// Tile x's softmax step (consume_tile's): its P^T operand; a raised reference rescales the accumulators, which by
// then hold tile x - 1's products too (the reference they were computed against is the old one).
template <int D, typename T>
E4_DEV u32x4_t softmax_phase(f32x4_t (&s)[2], f32x4_t (&acc)[D / 16], float& mref, float& lsum, float scale_log2,
                             uint32_t vis, bool full, int g) {
  constexpr float kSlack = 16.0f;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) s[kt][i] *= scale_log2;
  if (!full) {
    asm volatile("");
    const uint32_t vv = vis >> (4 * g);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) s[kt][i] = ((vv >> (16 * kt + i)) & 1u) ? s[kt][i] : -INFINITY;
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[kt][i]);
  if (__any(tmax > mref + kSlack)) {
    float rm = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    rm = fmaxf(rm, __shfl_xor(rm, 32, 64));
    const float m_new = fmaxf(mref, rm);
    const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mref - m_new);
    mref = m_new;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] *= alpha;
  }
  const float ref = mref == -INFINITY ? 0.f : mref;
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float p0 = __builtin_amdgcn_exp2f(s[p >> 1][2 * (p & 1)] - ref);
    const float p1 = __builtin_amdgcn_exp2f(s[p >> 1][2 * (p & 1) + 1] - ref);
    lsum += p0 + p1;
    w[p] = pack2<T>(p0, p1);
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

// The consumer step for an fp8 context tile (64 keys, two 32-key halves at K / V + 32 h D): the same schedule over
// both halves at once — the four S^T chains (half, kt) in flight together, one softmax step over the 64 scores — with
// the operands widened from fp8 as they are read and the per-(page, KV head) scales folded in per key: into the
// scores (s_k q . k8) and into P^T (p s_v, whose sum over keys stays the unscaled softmax denominator), so the
// products run on the exact e4m3 values. `scl` holds the tile's K scales (keys 0 .. 63) then its V scales.
template <int D, typename T>
E4_DEV void consume_tile_fp8(uint32_t kst, uint32_t vst, const OperandOffsets8& off, const u32x4_t (&q)[D / 32],
                             f32x4_t (&acc)[D / 16], float& mref, float& lsum, float scale_log2, uint32_t vis0,
                             uint32_t vis1, bool full, int g, const float4* scl) {
  constexpr float kSlack = 16.0f;
  constexpr int KG = 2, VG = 4;
  constexpr uint32_t kHalf = 32 * D;  // bytes from a half's rows to the next half's
  f32x4_t s[2][2];  // [half][kt]
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) s[h][kt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c0 = 0; c0 < D / 32; c0 += KG) {
    uint2 kraw[2][2][KG];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int c = 0; c < KG && c0 + c < D / 32; ++c) {
          const int cc = c0 + c;
          kraw[h][kt][c] = lds_load8(kst + off.kb[kt][cc & 3] + kHalf * h + 128 * (cc >> 2));
        }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int c = 0; c < KG && c0 + c < D / 32; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
          s[h][kt] = mfma16<T>(__builtin_bit_cast(u32x4_t, widen_fp8x8<T>(kraw[h][kt][c])), q[c0 + c], s[h][kt]);
  }
  uint32_t vb[8];  // the V reads' bases (at D 256 opaque, so that the half and 128 (dt / 8) stay in the offset field)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    vb[e] = off.vb[e];
    if constexpr (D == 256) {
      vb[e] += vst;
      asm volatile("" : "+v"(vb[e]));
    }
  }
  const uint32_t vsb = D == 256 ? 0u : vst;
  auto read_v = [&](int h, int dt) { return lds_tr8(vsb + vb[dt & 7] + kHalf * h + 128 * (dt >> 3)); };
  uint2 vop[VG];
#pragma unroll
  for (int i = 0; i < VG && i < D / 16; ++i) vop[i] = read_v(0, i);
  asm volatile("" ::: "memory");

  // scores in the log2 domain: key 32 h + 16 kt + 4 g + i takes its page's K scale
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      const float4 k4 = scl[8 * h + 4 * kt + g];
      const float ksc[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) s[h][kt][i] *= scale_log2 * ksc[i];
    }
  if (!full) {  // a tile with keys past the context
    asm volatile("");  // a branch, not selects
    const uint32_t vv[2] = {vis0 >> (4 * g), vis1 >> (4 * g)};
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[h][kt][i] = ((vv[h] >> (16 * kt + i)) & 1u) ? s[h][kt][i] : -INFINITY;
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) tmax = fmaxf(tmax, s[h][kt][i]);
  if (__any(tmax > mref + kSlack)) {
    float rm = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    rm = fmaxf(rm, __shfl_xor(rm, 32, 64));
    const float m_new = fmaxf(mref, rm);
    const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(mref - m_new);
    mref = m_new;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] *= alpha;
  }
  const float ref = mref == -INFINITY ? 0.f : mref;
  u32x4_t pb[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {  // element i of P^T's operand is key 16 (i / 4) + 4 g + i % 4 of the half
      const float4 v4 = scl[16 + 8 * h + 4 * kt + g];
      const float p0 = __builtin_amdgcn_exp2f(s[h][kt][0] - ref), p1 = __builtin_amdgcn_exp2f(s[h][kt][1] - ref);
      const float p2 = __builtin_amdgcn_exp2f(s[h][kt][2] - ref), p3 = __builtin_amdgcn_exp2f(s[h][kt][3] - ref);
      lsum += (p0 + p1) + (p2 + p3);
      pb[h][2 * kt] = pack2<T>(p0 * v4.x, p1 * v4.y);
      pb[h][2 * kt + 1] = pack2<T>(p2 * v4.z, p3 * v4.w);
    }
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int d0 = 0; d0 < D / 16; d0 += VG) {
      // the next group's V reads: this half's next d-tiles, or the second half's first
      const bool last = d0 + VG >= D / 16;
      uint2 nxt[VG];
      if (!(last && h == 1)) {
#pragma unroll
        for (int i = 0; i < VG && i < D / 16; ++i) nxt[i] = last ? read_v(1, i) : read_v(h, d0 + VG + i);
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int i = 0; i < VG && d0 + i < D / 16; ++i)
        acc[d0 + i] = mfma16<T>(__builtin_bit_cast(u32x4_t, widen_fp8x8<T>(vop[i])), pb[h], acc[d0 + i]);
      if (!(last && h == 1)) {
#pragma unroll
        for (int i = 0; i < VG && i < D / 16; ++i) vop[i] = nxt[i];
      }
    }
}

// Visible keys of a tile for one row: context tiles, positions below the context length; draft tiles, draft rows
// below the width whose ancestor bit the row holds.
E4_DEV uint32_t visible(bool is_new, int base, int hi, int width, int64_t row_mask) {
  const int n = is_new ? width - base : hi - base;
  const uint32_t below = n >= 32 ? 0xffffffffu : (n <= 0 ? 0u : (1u << n) - 1u);
  return is_new ? below & static_cast<uint32_t>(static_cast<uint64_t>(row_mask) >> base) : below;
}

// A producer's wait before handing tile x over: the loads it issued after tile x's are `later` tiles of NL direct
// loads plus, for the producer that runs the page lookups (LK = 1), S - 2 lookups.
template <int NS, int NL, int LK>
E4_DEV void wait_producer(int later) {
  static_assert(NS == 4, "waits written for four stages");
  constexpr int c0 = LK * (NS - 2), c1 = NL + LK * (NS - 2), c2 = 2 * NL + LK * (NS - 2);
  static_assert(c2 < 64, "vmcnt field");
  if (later >= 2)
    wait_vm<c2>();
  else if (later == 1)
    wait_vm<c1>();
  else
    wait_vm<c0>();
}

// vmcnt(n) for a count known only at run time (fp8 streams: a context tile and a draft tile issue different numbers
// of direct loads): a jump over immediate forms.
#define E4_WAIT_CASE(n) \
  case n:               \
    wait_vm<n>();       \
    break;
E4_DEV void wait_vm_dyn(int n) {
  switch (n) {
    E4_WAIT_CASE(1) E4_WAIT_CASE(2) E4_WAIT_CASE(3) E4_WAIT_CASE(4) E4_WAIT_CASE(5) E4_WAIT_CASE(6) E4_WAIT_CASE(7)
    E4_WAIT_CASE(8) E4_WAIT_CASE(9) E4_WAIT_CASE(10) E4_WAIT_CASE(11) E4_WAIT_CASE(12) E4_WAIT_CASE(13)
    E4_WAIT_CASE(14) E4_WAIT_CASE(15) E4_WAIT_CASE(16) E4_WAIT_CASE(17) E4_WAIT_CASE(18) E4_WAIT_CASE(19)
    E4_WAIT_CASE(20) E4_WAIT_CASE(21) E4_WAIT_CASE(22) E4_WAIT_CASE(23) E4_WAIT_CASE(24) E4_WAIT_CASE(25)
    E4_WAIT_CASE(26) E4_WAIT_CASE(27) E4_WAIT_CASE(28) E4_WAIT_CASE(29) E4_WAIT_CASE(30) E4_WAIT_CASE(31)
    E4_WAIT_CASE(32) E4_WAIT_CASE(33) E4_WAIT_CASE(34) E4_WAIT_CASE(35) E4_WAIT_CASE(36) E4_WAIT_CASE(37)
    E4_WAIT_CASE(38) E4_WAIT_CASE(39) E4_WAIT_CASE(40) E4_WAIT_CASE(41) E4_WAIT_CASE(42) E4_WAIT_CASE(43)
    E4_WAIT_CASE(44) E4_WAIT_CASE(45) E4_WAIT_CASE(46) E4_WAIT_CASE(47) E4_WAIT_CASE(48) E4_WAIT_CASE(49)
    E4_WAIT_CASE(50) E4_WAIT_CASE(51) E4_WAIT_CASE(52) E4_WAIT_CASE(53) E4_WAIT_CASE(54) E4_WAIT_CASE(55)
    E4_WAIT_CASE(56) E4_WAIT_CASE(57) E4_WAIT_CASE(58) E4_WAIT_CASE(59) E4_WAIT_CASE(60) E4_WAIT_CASE(61)
    E4_WAIT_CASE(62)
    default:
      wait_vm<0>();  // 0, and anything the field cannot hold: waiting for everything is always correct
  }
}
#undef E4_WAIT_CASE

// The rows of a finished piece, with the same stores on every path (no branch): normalised rows of dtype T to `out`
// (ooff: the lane's row from obase, in bytes) when the segment ends here, else fp32 partials normalised by their own
// sum and their log2-sum-exp to the workspace (poff / loff: the lane's partial row and lse word). A store that does not
// apply — the other kind, a lane without a row, the lse from lanes g != 0 — is addressed past its buffer's range
// (offset kDropped, or a range of zero bytes) and dropped. A fixed store count after the next segment's query loads lets
// the compiler wait for exactly those loads, where a branch on the kind made it wait for every store (vmcnt(0)).
constexpr uint32_t kDropped = 0x7ffffff0u;

template <int D, typename T>
E4_DEV void store_piece(const f32x4_t (&acc)[D / 16], float ls, float mref, bool fin, uint16_t* obase, uint32_t ooff,
                        float* pbase, uint32_t poff, float* lbase, uint32_t loff, int g) {
  const float inv = ls > 0.f ? 1.0f / ls : 0.f;
  const float lse = ls > 0.f ? mref + log2f(ls) : -INFINITY;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(obase, 0, fin ? kDropped : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(pbase, 0, fin ? 0 : kDropped, 0x00020000);
  const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(lbase, 0, fin ? 0 : kDropped, 0x00020000);
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    const f32x4_t v = acc[dt] * inv;
    __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{pack2<T>(v[0], v[1]), pack2<T>(v[2], v[3])}, ro,
                                          ooff + 2 * (16 * dt + 4 * g), 0, 2);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), rp, poff + 4 * (16 * dt + 4 * g), 0, 2);
  }
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse), rl, loff, 0, 2);
}

constexpr int waves_per_eu(int d) { return d == 256 ? 2 : (d == 128 ? 3 : 4); }

// One workgroup: C consumer waves (16 query rows each) and kProducers producer waves (page lookups, direct loads).
// FP8: context pages are fp8-e4m3 with per-(page, KV head) fp32 scales (draft rows stay 16-bit).
template <int D, int C, typename T, bool FP8>
__global__ __launch_bounds__(64 * (C + kProducers)) __attribute__((amdgpu_waves_per_eu(waves_per_eu(D))))
void verify_stream_kernel(const eagle4_attn_args a, const StreamPlan p) {
  static_assert(D % 32 == 0 && D >= 32 && D <= 256, "head dim");
  using TL = Tile<D>;
  constexpr int NW = C + kProducers;
  constexpr int NT = 64 * NW;
  constexpr int NS = kStages;
  constexpr int NG = TL::NI / kProducers;  // row groups per producer: nn = producer + kProducers i, K then V
  constexpr int CK = FP8 ? kTileKeys8 : kTileKeys;  // keys of a context tile
  // Tiles the loads run ahead of the compute: the load of tile x + LD goes out when tile x is handed over. 16-bit pages
  // run their consumers pipelined (tile x - 1's PV products in iteration x), so stage x - 1 is still read then and the
  // loads stay two tiles ahead; fp8 pages keep three. Page lookups run NS - 1 tiles ahead of the loads.
  constexpr bool kPipe = !FP8;
  constexpr int LD = kPipe ? NS - 2 : NS - 1;
  static_assert(TL::NI % kProducers == 0, "row groups split evenly");
  __shared__ __attribute__((aligned(1024))) char smem[NS][2][TL::BYTES];  // [stage][K, V]
  __shared__ __attribute__((aligned(256))) int s_pid[NS][64];             // page ids of a tile's keys
  __shared__ int s_qsl[kStreamMaxReqs + 1];
  __shared__ int s_ctx[kStreamMaxReqs];
  __shared__ int64_t s_wsum[NW];
  __shared__ int64_t s_start[2];
  __shared__ int64_t s_share[2];  // this share's first tile and the next share's
  __shared__ __attribute__((aligned(16))) float s_scl[FP8 ? NS : 1][2 * kTileKeys8];  // fp8: K, V scales per key

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = uni(tid >> 6);
  // Roles. Waves go to the CU's four SIMDs round-robin (wave w on SIMD w % 4). With six consumers on 16-bit pages the
  // producers take waves 0 and 4, a SIMD of their own, so their issue never queues behind consumer MFMA and VALU
  // work (per-tile interval 1.57 -> 1.45 us at batch 64); fp8 consumers are VALU-bound and keep all four SIMDs.
  constexpr bool kOwnSimd = C == 6 && !FP8;
  const bool producer = kOwnSimd ? (wave & 3) == 0 : wave >= C;
  const int cw = kOwnSimd ? (wave >> 2) * 3 + (wave & 3) - 1 : wave;  // consumer index (producers: unused)
  const int g = lane >> 4, l16 = lane & 15;
  const int B = a.num_reqs;
  const int HR = p.HR;

  // ---- the requests' query starts and (clamped) contexts, and each workgroup's share of the tile sequence ------
  {
    const int64_t capacity = static_cast<int64_t>(a.max_blocks) * a.page;
    for (int i = tid; i <= B; i += NT) s_qsl[i] = static_cast<int>(e4::ld(a.query_start_loc, i));
    for (int i = tid; i < B; i += NT) {
      const int64_t c = e4::ld(a.context_lens, i);
      s_ctx[i] = static_cast<int>(c < 0 ? 0 : (c > capacity ? capacity : c));
    }
  }
  __syncthreads();
  // Shares split the sequence by cost, not by tiles: a tile costs 4 units and a segment's end (its rows stored, the
  // next segment's loaded) p.seg_cost more, so that shares holding more segment ends hold fewer tiles. Each thread
  // takes a range of requests; (tiles | non-empty requests << 40) is scanned over the workgroup.
  constexpr int kCnt = 40;
  constexpr int64_t kTileMask = (int64_t(1) << kCnt) - 1;
  const int per = (B + NT - 1) / NT;
  const int b_lo = tid * per < B ? tid * per : B;
  const int b_hi = b_lo + per < B ? b_lo + per : B;
  int64_t mine = 0;
  for (int b = b_lo; b < b_hi; ++b) {
    const int tb = tiles_of<CK>(s_qsl, s_ctx, b);
    mine += tb + (tb > 0 ? int64_t(1) << kCnt : 0);
  }
  int64_t incl = mine;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) s_wsum[wave] = incl;
  __syncthreads();
  int64_t before = incl - mine, total = 0;
#pragma unroll
  for (int w2 = 0; w2 < NW; ++w2) {
    const int64_t v = s_wsum[w2];
    before += w2 < wave ? v : 0;
    total += v;
  }
  const int64_t total_t = total & kTileMask;
  const int64_t tiles_all = total_t * HR;
  const int64_t nact = active_groups(tiles_all, p.nwg);
  const int64_t E = p.seg_cost;
  const int64_t cost_all = HR * (4 * total_t + E * (total >> kCnt));
  const int w = blockIdx.x;
  const int64_t c0 = nact > 0 ? cost_all * w / nact : 0, c1 = nact > 0 ? cost_all * (w + 1) / nact : 0;
  int64_t* const pre = reinterpret_cast<int64_t*>(a.workspace);  // [B + 1] tiles before each request, then shares
  {
    int64_t run_t = before & kTileMask, run_n = before >> kCnt;
    for (int b = b_lo; b < b_hi; ++b) {
      const int tb = tiles_of<CK>(s_qsl, s_ctx, b);
      if (w == 0) pre[b] = run_t;
      if (tb > 0) {
        const int64_t cb = HR * (4 * run_t + E * run_n), sc = 4 * tb + E;  // cost before b; of one of its segments
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int64_t c = i == 0 ? c0 : c1;
          if (cb <= c && c < cb + HR * sc) {  // the first tile at or past cost c; past a segment's last tile: the next
            const int64_t k = (c - cb) / sc, u = c - cb - k * sc;
            s_share[i] = run_t * HR + (u > 4 * (tb - 1) ? (k + 1) * tb : k * tb + (u + 3) / 4);
          }
        }
        run_t += tb;
        run_n += 1;
      }
    }
    if (w == 0 && tid == 0) pre[B] = total_t;
  }
  __syncthreads();
  const int64_t g0 = c0 < cost_all ? s_share[0] : tiles_all;
  const int64_t g1 = c1 < cost_all ? s_share[1] : tiles_all;
  {
    int64_t run = before & kTileMask;
    for (int b = b_lo; b < b_hi; ++b) {
      const int tb = tiles_of<CK>(s_qsl, s_ctx, b);
      if (tb > 0 && run * HR <= g0 && g0 < (run + tb) * HR) {
        s_start[0] = b;
        s_start[1] = run;
      }
      run += tb;
    }
  }
  __syncthreads();
  if (w >= nact || g0 >= g1) return;

  // ---- cursors: compute (cc), direct loads (cd, S - 1 ahead), page lookups (cl, 2 S - 2 ahead) -------------------
  Cursor cc;
  {
    cc.b = uni(static_cast<int>(s_start[0]));
    cur_load<CK>(cc, s_qsl, s_ctx, B);
    const int64_t off = g0 - s_start[1] * HR;
    cc.k = uni(static_cast<int>(off / cc.tiles));
    cc.j = uni(static_cast<int>(off - static_cast<int64_t>(cc.k) * cc.tiles));
  }
  const int RG = p.RG;

  if (producer) {  // ---- producers ---------------------------------------------------------------------------------
    const int pi = kOwnSimd ? wave >> 2 : wave - C;  // producer 0 also runs the page lookups
    Cursor cd = cc, cl = cc;
    const int page = a.page;
    const int page_shift = (page & (page - 1)) == 0 ? __builtin_ctz(page) : -1;
    const char* const kcache = static_cast<const char*>(a.key_cache);
    const char* const vcache = static_cast<const char*>(a.value_cache);
    constexpr int EB = FP8 ? 1 : 2;  // bytes per cache element
    const int64_t kb2 = a.stride_kb * EB, ks2 = a.stride_ks * EB, kh2 = a.stride_kh * EB;
    const int64_t vb2 = a.stride_vb * EB, vs2 = a.stride_vs * EB, vh2 = a.stride_vh * EB;
    const char* const knew = static_cast<const char*>(a.k_new);
    const char* const vnew = static_cast<const char*>(a.v_new);
    const int64_t knt2 = a.stride_knt * 2, knh2 = a.stride_knh * 2, vnt2 = a.stride_vnt * 2, vnh2 = a.stride_vnh * 2;
    const int32_t* const bt = static_cast<const int32_t*>(a.block_table.ptr);
    const int32_t* const bt_dummy = static_cast<const int32_t*>(a.query_start_loc.ptr);  // any readable word
    const int pc = lane % TL::CH, lrow = lane / TL::CH;
    // direct pages: lane offsets of this producer's row group i (nn = pi + kProducers i) from the start of its page
    // (pages that are multiples of the context tile hold the whole tile: its first slot is added to the page base)
    const bool whole = page % CK == 0;
    uint32_t koff[NG], voff[NG];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int r0 = (pi + kProducers * i) * TL::RPI;
      const int slot_row = (whole ? r0 : (r0 & (page - 1))) + lrow;
      koff[i] = static_cast<uint32_t>(slot_row * ks2 + 16 * (pc ^ TL::kswz(r0 + lrow)));
      voff[i] = static_cast<uint32_t>(slot_row * vs2 + 16 * (pc ^ TL::vswz(r0 + lrow)));
    }
    const uint32_t kbu = static_cast<uint32_t>(kb2), vbu = static_cast<uint32_t>(vb2);
    // fp8 context tiles: rows of D bytes, instructions nn = pi + kProducers i below Tile8::NI (RPI8 rows each)
    using T8 = Tile8<D>;
    constexpr int NG8 = (T8::NI + kProducers - 1) / kProducers;
    const int pc8 = lane % T8::CH, lrow8 = lane / T8::CH;
    uint32_t koff8[NG8], voff8[NG8];
#pragma unroll
    for (int i = 0; i < NG8; ++i) {
      const int r0 = (pi + kProducers * i) * T8::RPI;
      const int slot_row = (whole ? r0 : (r0 & (page - 1))) + lrow8;
      koff8[i] = static_cast<uint32_t>(slot_row * ks2 + 16 * (pc8 ^ T8::kswz(r0 + lrow8)));
      voff8[i] = static_cast<uint32_t>(slot_row * vs2 + 16 * (pc8 ^ T8::vswz(r0 + lrow8)));
    }
    const int mine8 = (T8::NI - pi + kProducers - 1) / kProducers;  // fp8 instructions of this producer per matrix
    // the direct loads a tile makes this producer issue (K and V, plus the scales' for producer 0 on fp8 pages)
    auto loads_of = [&](const Cursor& c) {
      if (FP8 && c.j < c.n_ctx) return 2 * mine8 + (pi == 0 ? 2 : 0);
      return 2 * NG;
    };

    // page ids of tile c's keys into ring slot `slot` (draft tiles and look-ahead past the end: a dummy read, so
    // every iteration issues the same loads)
    auto lookup = [&](const Cursor& c, int slot) {
      if (pi != 0) return;
      const int32_t* src = bt_dummy;
      if (c.j < c.n_ctx) {
        const int base = c.j * CK;
        const int first = page_div(base, page, page_shift);
        const int last = page_div(base + CK - 1 < c.ctx ? base + CK - 1 : c.ctx - 1, page, page_shift);
        const int idx = first + lane < last ? first + lane : last;
        src = bt + static_cast<int64_t>(c.b) * a.block_table.s0 + idx;
      }
      dma4(src, uni(lds_addr(s_pid[slot])));
    };
    // this producer's share of tile c's K / V into stage `slot`: row groups nn = pi + kProducers i (rows RPI nn ..
    // RPI nn + RPI - 1), K then V
    auto load_tile = [&](const Cursor& c, int slot) {
      const int kvh = c.k / RG;
      const uint32_t kl = lds_addr(smem[slot][0]), vl = lds_addr(smem[slot][1]);
      if (c.j < c.n_ctx) {
        const int base = c.j * CK;
        const int first = page_div(base, page, page_shift);
        const char* const kh = kcache + kvh * kh2;
        const char* const vh = vcache + kvh * vh2;
        if constexpr (FP8) {
          if (pi == 0) {  // the scales of the tile's 64 keys, K then V (keys past the context take the last one's)
            const int pos = base + lane < c.ctx ? base + lane : c.ctx - 1;
            const int64_t pid = s_pid[slot][page_div(pos, page, page_shift) - first];
            dma4(a.k_scale + pid * a.stride_ksb + kvh * a.stride_ksh, uni(lds_addr(s_scl[slot])));
            dma4(a.v_scale + pid * a.stride_vsb + kvh * a.stride_vsh, uni(lds_addr(s_scl[slot] + 64)));
          }
          if (p.direct) {
            const int ids = s_pid[slot][lane];
            const int in0 = whole ? base - first * page : 0;
            const char* const kt = kh + in0 * ks2;
            const char* const vt = vh + in0 * vs2;
#pragma unroll
            for (int i = 0; i < NG8; ++i) {
              const int nn = pi + kProducers * i;
              if (nn < T8::NI) {
                const int rel = whole ? 0 : (nn * T8::RPI) >> page_shift;
                const uint32_t pid = static_cast<uint32_t>(__builtin_amdgcn_readlane(ids, rel));
                dma16s(kt + static_cast<uint64_t>(pid) * kbu, koff8[i], uni(kl + nn * 1024));
                dma16s(vt + static_cast<uint64_t>(pid) * vbu, voff8[i], uni(vl + nn * 1024));
              }
            }
          } else {
#pragma unroll
            for (int i = 0; i < NG8; ++i) {
              const int nn = pi + kProducers * i;
              if (nn < T8::NI) {
                const int row = nn * T8::RPI + lrow8;
                const int pos = base + row < c.ctx ? base + row : c.ctx - 1;
                const int pg = page_div(pos, page, page_shift);
                const int64_t pid = s_pid[slot][pg - first];
                const int64_t sl = pos - pg * page;
                dma16(kh + pid * kb2 + sl * ks2 + 16 * (pc8 ^ T8::kswz(row)), uni(kl + nn * 1024));
                dma16(vh + pid * vb2 + sl * vs2 + 16 * (pc8 ^ T8::vswz(row)), uni(vl + nn * 1024));
              }
            }
          }
        } else if (p.direct) {
          // a row group lies in one page (rows past the context read the last page's slots: in bounds, masked); the
          // tile's page ids come from one LDS read, lane i holding the id of page first + i
          const int ids = s_pid[slot][lane];
          const int in0 = whole ? base - first * page : 0;
          const char* const kt = kh + in0 * ks2;
          const char* const vt = vh + in0 * vs2;
#pragma unroll
          for (int i = 0; i < NG; ++i) {
            const int nn = pi + kProducers * i;
            const int rel = whole ? 0 : (nn * TL::RPI) >> page_shift;  // pages below 32 keys: powers of two
            const uint32_t pid = static_cast<uint32_t>(__builtin_amdgcn_readlane(ids, rel));
            dma16s(kt + static_cast<uint64_t>(pid) * kbu, koff[i], uni(kl + nn * 1024));
            dma16s(vt + static_cast<uint64_t>(pid) * vbu, voff[i], uni(vl + nn * 1024));
          }
        } else {
#pragma unroll
          for (int i = 0; i < NG; ++i) {
            const int nn = pi + kProducers * i;
            const int row = nn * TL::RPI + lrow;
            const int pos = base + row < c.ctx ? base + row : c.ctx - 1;  // past the context: its last key (masked)
            const int pg = page_div(pos, page, page_shift);
            const int64_t pid = s_pid[slot][pg - first];
            const int64_t sl = pos - pg * page;
            const char* ksrc = kh + pid * kb2 + sl * ks2 + 16 * (pc ^ TL::kswz(row));
            const char* vsrc = vh + pid * vb2 + sl * vs2 + 16 * (pc ^ TL::vswz(row));
            dma16(ksrc, uni(kl + nn * 1024));
            dma16(vsrc, uni(vl + nn * 1024));
          }
        }
      } else {
        const int base = (c.j - c.n_ctx) * kTileKeys;
#pragma unroll
        for (int i = 0; i < NG; ++i) {
          const int nn = pi + kProducers * i;
          const int row = nn * TL::RPI + lrow;
          const int key = base + row < c.width ? base + row : c.width - 1;  // past the draft rows: the last (masked)
          const int64_t tok = c.qs + key;
          const char* ksrc = knew + tok * knt2 + kvh * knh2 + 16 * (pc ^ TL::kswz(row));
          const char* vsrc = vnew + tok * vnt2 + kvh * vnh2 + 16 * (pc ^ TL::vswz(row));
          dma16(ksrc, uni(kl + nn * 1024));
          dma16(vsrc, uni(vl + nn * 1024));
        }
      }
    };

    // prologue (kStages barriers, matched by the consumers): lookups of the first S - 1 tiles, landed before any
    // producer reads them; then those tiles' loads interleaved with the next lookups in the steady state's order, a
    // barrier after each step (a lookup reuses the ring slot that both producers read in the step before)
    for (int i = 0; i < NS - 1; ++i) {
      lookup(cl, static_cast<int>((g0 + i) & (NS - 1)));
      cur_next<CK>(cl, s_qsl, s_ctx, B, HR);
    }
    wait_vm<0>();
    __syncthreads();
    static_assert(NS == 4, "the load-count window below is written for four stages");
    int n1 = 0, n2 = 0;  // fp8: direct loads of tiles x + 1 and x + 2 (tiles differ: fp8 context, 16-bit draft)
    for (int i = 0; i < LD; ++i) {
      int n = 0;
      if (g0 + i < g1) {
        n = loads_of(cd);
        load_tile(cd, static_cast<int>((g0 + i) & (NS - 1)));
      }
      if (i == 1) n1 = n;
      if (i == 2) n2 = n;
      cur_next<CK>(cd, s_qsl, s_ctx, B, HR);
      lookup(cl, static_cast<int>((g0 + NS - 1 + i) & (NS - 1)));
      cur_next<CK>(cl, s_qsl, s_ctx, B, HR);
      __syncthreads();
    }
    for (int64_t x = g0; x < g1; ++x) {
      const int slot = static_cast<int>(x & (NS - 1));
      const int64_t left = g1 - x - 1;
      const int later = static_cast<int>(left < LD - 1 ? left : LD - 1);
      if constexpr (FP8) {  // loads issued after tile x's: those of the later tiles and the lookups 4, 5 ahead
        wait_vm_dyn((later >= 1 ? n1 : 0) + (later >= 2 ? n2 : 0) + (pi == 0 ? NS - 2 : 0));
      } else if (pi == 0) {
        wait_producer<NS, 2 * NG, 1>(later);
      } else {
        wait_producer<NS, 2 * NG, 0>(later);
      }
      __syncthreads();  // tile x is in LDS; stage x - LD + 1 ... x - 1 ... has been read by every consumer
      int n3 = 0;
      if (x + LD < g1) {
        n3 = loads_of(cd);
        load_tile(cd, (slot + LD) & (NS - 1));
      }
      n1 = n2;
      n2 = n3;
      cur_next<CK>(cd, s_qsl, s_ctx, B, HR);
      lookup(cl, (slot + LD + NS - 1) & (NS - 1));
      cur_next<CK>(cl, s_qsl, s_ctx, B, HR);
    }
    wait_vm<0>();
    return;
  }

  // ---- consumers ---------------------------------------------------------------------------------------------------
  const int G = p.G;
  const float scale_log2 = a.scale * 1.4426950408889634f;
  u32x4_t q[D / 32];
  int64_t row_mask = 0;
  bool row_ok = false;
  int t = 0, head = 0;
  // the segment's row of this lane: Q, ancestor mask
  auto enter = [&](const Cursor& c, u32x4_t (&qr)[D / 32], int64_t& mask_r, bool& ok_r, int& t_r, int& head_r) {
    const int kvh = c.k / RG, rg = c.k - kvh * RG;
    const int rows = c.width < a.max_query_len ? c.width : a.max_query_len;
    const int rt = rg * C + cw;
    const int rho = rt * 16 + l16;
    t_r = rho / G;
    head_r = kvh * G + (rho - t_r * G);
    ok_r = rt < p.row_tiles && t_r < rows;
    load_q<D>(qr, static_cast<const uint16_t*>(a.q) + (c.qs + t_r) * a.stride_qt + head_r * a.stride_qh, ok_r, g);
    mask_r = ok_r ? a.masks[static_cast<int64_t>(c.b) * a.stride_mask + t_r] : 0;
  };
  enter(cc, q, row_mask, row_ok, t, head);
  f32x4_t acc[D / 16];
  float mref, lsum;
  auto reset = [&] {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    mref = -INFINITY;
    lsum = 0.f;
  };
  reset();
  const OperandOffsets off = operand_offsets<D>(g, l16);
  OperandOffsets8 off8 = {};
  if constexpr (FP8) off8 = operand_offsets8<D>(g, l16);
  int piece_j0 = cc.j;
  const int rows_seg = p.rows_seg;
  // 16-bit pages: the next segment's rows are loaded kAheadTiles tiles before this segment ends, into qn / mask_n.
  // Loaded at the end, they waited behind the K / V stream this CU has in flight (~2 us per segment end).
  constexpr bool kPrefetch = !FP8;
  u32x4_t qn[kPrefetch ? D / 32 : 1];
  int64_t mask_n = 0;
  bool ok_n = false, fetched = false;
  int t_n = 0, head_n = 0;
  Cursor cn = cc;
  // tiles whose keys are all visible skip the mask (at D 256; smaller heads have no registers to spare for it)
  constexpr bool kFullTiles = D == 256;
  // pipelined consumers: tile x - 1's P^T and stage, its PV products still to run
  bool pend = false;
  int prev = 0;
  u32x4_t pb = {0u, 0u, 0u, 0u};
  // the first rows' loads waited for here, so that the loop's wait for a segment's rows (loaded before the previous
  // piece's stores) is not merged with a wait made for these
#pragma unroll
  for (int i = 0; i < D / 32; ++i) asm volatile("" ::"v"(q[i]));
  asm volatile("" ::"v"(row_mask));
#pragma unroll
  for (int i = 0; i < LD + 1; ++i) __syncthreads();  // the producers' prologue

  for (int64_t x = g0; x < g1; ++x) {
    const int slot = static_cast<int>(x & (NS - 1));
    __syncthreads();
    if constexpr (kPrefetch) {
      if (!fetched && cc.tiles - 1 - cc.j <= kAheadTiles && x + (cc.tiles - cc.j) < g1) {  // the next segment is ours
        cn = cc;
        cn.j = cn.tiles - 1;
        cur_next<CK>(cn, s_qsl, s_ctx, B, HR);
        enter(cn, qn, mask_n, ok_n, t_n, head_n);
        fetched = true;
      }
    }
    const bool is_new = cc.j >= cc.n_ctx;
    const int base = is_new ? (cc.j - cc.n_ctx) * kTileKeys : cc.j * CK;
    if (FP8 && !is_new) {  // the 64-key fp8 tile
      consume_tile_fp8<D, T>(lds_addr(smem[slot][0]), lds_addr(smem[slot][1]), off8, q, acc, mref, lsum, scale_log2,
                             visible(false, base, cc.ctx, cc.width, row_mask),
                             visible(false, base + 32, cc.ctx, cc.width, row_mask),
                             kFullTiles && base + kTileKeys8 <= cc.ctx, g,
                             reinterpret_cast<const float4*>(s_scl[FP8 ? slot : 0]));
    } else if constexpr (kPipe) {
      f32x4_t sx[2];
      qk_phase<D, T>(lds_addr(smem[slot][0]), off, q, sx);
      if (pend) pv_phase<D, T>(lds_addr(smem[prev][0]), off, pb, acc);  // tile x - 1's, behind the QK products
      pb = softmax_phase<D, T>(sx, acc, mref, lsum, scale_log2, visible(is_new, base, cc.ctx, cc.width, row_mask),
                               kFullTiles && !is_new && base + kTileKeys <= cc.ctx, g);
      pend = true;
      prev = slot;
    } else {
      consume_tile<D, T>(lds_addr(smem[slot][0]), off, q, acc, mref, lsum, scale_log2,
                         visible(is_new, base, cc.ctx, cc.width, row_mask),
                         kFullTiles && !is_new && base + kTileKeys <= cc.ctx, g);
    }

    const bool seg_end = cc.j == cc.tiles - 1;
    if ((cc.j == 0 || seg_end) && cw == 0) {  // the shares holding the segment's first and last tiles (every lane
                                               // stores the same word: no lane branch inside the loop)
      int32_t* const seg_w = reinterpret_cast<int32_t*>(pre + B + 1) + 2 * (static_cast<int64_t>(cc.b) * HR + cc.k);
      if (cc.j == 0) seg_w[0] = w;
      if (seg_end) seg_w[1] = w;
    }
    if (seg_end || x == g1 - 1) {
      if constexpr (kPipe) {  // the piece's last PV products
        pv_phase<D, T>(lds_addr(smem[slot][0]), off, pb, acc);
        pend = false;
      }
      const bool more = x + 1 < g1;
      float ls = lsum + __shfl_xor(lsum, 16, 64);
      ls += __shfl_xor(ls, 32, 64);
      // where this piece's rows go: a segment finished here to `out`; a piece of a cut segment to slot 2 w (the share's
      // first piece, it starts inside a segment) or 2 w + 1 (its last, it ends inside one)
      const bool fin = piece_j0 == 0 && seg_end;
      uint16_t* const obase = static_cast<uint16_t*>(a.out) + cc.qs * a.stride_ot;
      const uint32_t ooff = row_ok ? static_cast<uint32_t>((t * a.stride_ot + head * a.stride_oh) * 2) : kDropped;
      const int64_t part = (piece_j0 > 0 ? 2 * w : 2 * w + 1) * static_cast<int64_t>(rows_seg) + 16 * cw + l16;
      const uint32_t poff = row_ok ? static_cast<uint32_t>(part * D * 4) : kDropped;
      const uint32_t loff = row_ok && g == 0 ? static_cast<uint32_t>(part * 4) : kDropped;
      // The next segment's rows: 16-bit pages prefetched them into qn (at the latest on this tile, so always when there
      // is a next segment); fp8 pages below D 128 load them here, straight into q and row_mask before this piece's
      // stores; fp8 pages at D >= 128 have no registers for q and the accumulators at once and load them after. A load
      // before the stores is waited for with the stores' count (vmcnt retires in issue order), not behind them; the
      // branch-free stores keep that count the same on every path.
      constexpr bool kAhead = !FP8 || D < 128;
      if (!kPrefetch && kAhead && more) {
        cur_next<CK>(cc, s_qsl, s_ctx, B, HR);
        enter(cc, q, row_mask, row_ok, t, head);
      }
      if constexpr (kAhead) {
        store_piece<D, T>(acc, ls, mref, fin, obase, ooff, a.workspace + p.part_off, poff, a.workspace + p.lse_off,
                          loff, g);
      } else if (row_ok) {  // registers too short for the branch-free form; these waves wait for their stores anyway
        const float inv = ls > 0.f ? 1.0f / ls : 0.f;
        if (fin) {
          store_rows<D, T>(obase + t * a.stride_ot + head * a.stride_oh, acc, inv, g);
        } else {
          store_partial<D>(a.workspace + p.part_off + part * D, acc, inv, g);
          if (g == 0) a.workspace[p.lse_off + part] = ls > 0.f ? mref + log2f(ls) : -INFINITY;
        }
      }
      if (more) {
        if constexpr (kPrefetch) {
          cc = cn;
#pragma unroll
          for (int i = 0; i < D / 32; ++i) q[i] = qn[i];
          row_mask = mask_n;
          row_ok = ok_n;
          t = t_n;
          head = head_n;
          fetched = false;
        } else if constexpr (!kAhead) {
          cur_next<CK>(cc, s_qsl, s_ctx, B, HR);
          enter(cc, q, row_mask, row_ok, t, head);
        }
        reset();
        piece_j0 = 0;
      }
    } else {
      ++cc.j;
    }
  }
}

// Merges the pieces of each segment cut by share boundaries (vllm/verify_attention.py:115-139): weights
// 2^(lse_i - max) over the pieces' normalised fp32 partials. A thread takes 16 columns of one row and folds the pieces
// four at a time with a running max, every load of a group of four issued before the first is used.
template <int D, typename T>
__global__ __launch_bounds__(256) void verify_stream_merge(const eagle4_attn_args a, const StreamPlan p) {
  constexpr int kCols = D < 16 ? D : 16;
  constexpr int TPR = D / kCols;  // threads per row
  constexpr int NV = kCols / 4;   // float4 per thread and piece
  constexpr int kGroup = 4;       // pieces in flight
  const int s = blockIdx.x;
  const int b = s / p.HR, k = s - b * p.HR;
  const int64_t* pre = reinterpret_cast<const int64_t*>(a.workspace);
  const int64_t tiles = pre[b + 1] - pre[b];
  if (tiles <= 0) return;
  // the shares that computed the segment's first and last tiles (recorded by the stream kernel in this launch)
  const int32_t* const seg_w = reinterpret_cast<const int32_t*>(pre + a.num_reqs + 1) + 2 * static_cast<int64_t>(s);
  const int64_t w0 = seg_w[0], w1 = seg_w[1];
  if (w0 == w1) return;  // inside one share: written directly
  const int item = blockIdx.y * 256 + threadIdx.x;
  const int rows_seg = p.rows_seg;
  if (item >= rows_seg * TPR) return;
  const int r = item / TPR, d = kCols * (item % TPR);
  const int G = p.G, kvh = k / p.RG, rg = k - kvh * p.RG;
  const int64_t qs = e4::ld(a.query_start_loc, b);
  int64_t rows = e4::ld(a.query_start_loc, b + 1) - qs;
  rows = rows < a.max_query_len ? rows : a.max_query_len;
  const int rho = rg * rows_seg + r;
  const int rt = rho / 16;
  const int t = rho / G, gq = rho - t * G;
  if (rt >= p.row_tiles || t >= rows) return;
  float mx = -INFINITY, wsum = 0.f;
  float sum[kCols];
#pragma unroll
  for (int c = 0; c < kCols; ++c) sum[c] = 0.f;
  for (int64_t wg = w0; wg <= w1; wg += kGroup) {
    float ls[kGroup];
    float4 v[kGroup][NV];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      const bool in = wg + i <= w1;
      // share w0's piece is its last (slot 2 w0 + 1), every later share's its first (slot 2 w)
      const int64_t piece = in ? wg + i : w0;
      const int64_t part = (piece == w0 ? 2 * piece + 1 : 2 * piece) * rows_seg + r;
      ls[i] = in ? a.workspace[p.lse_off + part] : -INFINITY;
#pragma unroll
      for (int c = 0; c < NV; ++c)
        v[i][c] = in ? *reinterpret_cast<const float4*>(a.workspace + p.part_off + part * D + d + 4 * c)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < kGroup; ++i) {
      if (ls[i] == -INFINITY) continue;  // past the last piece, or a piece with no visible key
      const float m_new = fmaxf(mx, ls[i]);
      const float keep = exp2f(mx - m_new), wt = exp2f(ls[i] - m_new);
#pragma unroll
      for (int c = 0; c < NV; ++c) {
        sum[4 * c] = sum[4 * c] * keep + wt * v[i][c].x;
        sum[4 * c + 1] = sum[4 * c + 1] * keep + wt * v[i][c].y;
        sum[4 * c + 2] = sum[4 * c + 2] * keep + wt * v[i][c].z;
        sum[4 * c + 3] = sum[4 * c + 3] * keep + wt * v[i][c].w;
      }
      wsum = wsum * keep + wt;
      mx = m_new;
    }
  }
  const float inv = wsum > 0.f ? 1.0f / wsum : 0.f;
  uint16_t* orow = static_cast<uint16_t*>(a.out) + (qs + t) * a.stride_ot +
                   (static_cast<int64_t>(kvh) * G + gq) * a.stride_oh + d;
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    uint2 o;
    o.x = pack2<T>(sum[4 * c] * inv, sum[4 * c + 1] * inv);
    o.y = pack2<T>(sum[4 * c + 2] * inv, sum[4 * c + 3] * inv);
    *reinterpret_cast<uint2*>(orow + 4 * c) = o;
  }
}

template <int D, int C, typename T, bool FP8>
int resident_groups() {
  static const int per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(verify_stream_kernel<D, C, T, FP8>), 64 * (C + kProducers), 0) !=
        hipSuccess)
      n = 0;
    return n;
  }();
  int dev = 0, cus = 0;
  if (per_cu <= 0 || hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 0;
  return per_cu * cus;
}

template <int D, int C, typename T, bool FP8>
int launch(const eagle4_attn_args& a, const StreamPlan& p, hipStream_t s) {
  verify_stream_kernel<D, C, T, FP8><<<p.nwg, 64 * (C + kProducers), 0, s>>>(a, p);
  constexpr int kMergeThreadsPerRow = D / (D < 16 ? D : 16);
  verify_stream_merge<D, T><<<dim3(a.num_reqs * p.HR,
                                   e4::ceil_div(static_cast<int64_t>(p.rows_seg) * kMergeThreadsPerRow, 256)),
                              256, 0, s>>>(a, p);
  return E4_LAUNCH_STATUS();
}

// The instantiations: head dims 32 .. 256, 2 / 4 / 6 consumer waves (a group of row tiles takes the smallest that
// holds it), bf16 / fp16 rows, 16-bit or fp8 pages; `go` receives the one the call needs (as a type tag).
template <int D_, int C_, typename T_, bool FP8_>
struct Config {
  static constexpr int D = D_, C = C_;
  using T = T_;
  static constexpr bool FP8 = FP8_;
};

template <int D, typename T, bool FP8, typename F>
int with_c(int c, F&& go) {
  switch (c) {
    case 2: return go(Config<D, 2, T, FP8>{});
    case 4: return go(Config<D, 4, T, FP8>{});
    default: return go(Config<D, 6, T, FP8>{});
  }
}

template <int D, typename F>
int with_t(const eagle4_attn_args& a, int c, F&& go) {
  const bool bf = a.dtype == EAGLE4_BF16, f8 = a.cache_dtype == EAGLE4_FP8_E4M3;
  if (bf) return f8 ? with_c<D, e4::Bf16, true>(c, go) : with_c<D, e4::Bf16, false>(c, go);
  return f8 ? with_c<D, e4::F16, true>(c, go) : with_c<D, e4::F16, false>(c, go);
}

template <typename F>
int with_config(const eagle4_attn_args& a, int c, F&& go) {
  switch (a.D) {
    case 32: return with_t<32>(a, c, go);
    case 64: return with_t<64>(a, c, go);
    case 128: return with_t<128>(a, c, go);
    default: return with_t<256>(a, c, go);
  }
}

}  // namespace

// 16-bit caches of q's dtype, or fp8-e4m3 caches with their scales; at most kStreamMaxReqs requests; the library's
// context split (a caller-chosen split size selects the split-context schedule). The rest of the contract is checked
// by the caller.
bool stream_covered(const eagle4_attn_args& a) {
  const bool fp8 = a.cache_dtype == EAGLE4_FP8_E4M3 && a.k_scale != nullptr && a.v_scale != nullptr;
  // a request's output rows are addressed by 32-bit byte offsets from its first row (the branch-free stores)
  const int64_t span = (static_cast<int64_t>(a.max_query_len) * a.stride_ot + static_cast<int64_t>(a.Hq) * a.stride_oh +
                        a.D) * 2;
  const bool rows_ok = a.stride_ot >= 0 && a.stride_oh >= 0 && span < (int64_t(1) << 30);
  return (a.cache_dtype == a.dtype || fp8) && rows_ok && a.num_reqs <= kStreamMaxReqs && a.chunk <= 0 &&
         !small_attention_job(a);
}

bool stream_plan(const eagle4_attn_args& a, StreamPlan& p) {
  p.G = a.Hq / a.Hkv;
  p.row_tiles = e4::ceil_div(static_cast<int64_t>(p.G) * a.max_query_len, 16);
  p.RG = e4::ceil_div(p.row_tiles, 6);
  const int need = e4::ceil_div(p.row_tiles, p.RG);
  p.C = need <= 2 ? 2 : (need <= 4 ? 4 : 6);
  p.HR = a.Hkv * p.RG;
  p.rows_seg = 16 * p.C;
  p.fp8 = a.cache_dtype == EAGLE4_FP8_E4M3;
  // direct page addressing: every direct-load instruction's rows (1024 / (element bytes x D) consecutive keys) in one
  // page, a page's slots addressable by 32-bit lane offsets, block strides below 4 GB
  const int eb = p.fp8 ? 1 : 2;
  const int rpi = 1024 / (eb * a.D);
  const int ck = p.fp8 ? kTileKeys8 : kTileKeys;
  const bool aligned = a.page % ck == 0 || (ck % a.page == 0 && a.page >= rpi);
  const int64_t span = static_cast<int64_t>(a.page) * (a.stride_ks > a.stride_vs ? a.stride_ks : a.stride_vs) * eb;
  const int64_t block_bytes = eb * (a.stride_kb > a.stride_vb ? a.stride_kb : a.stride_vb);
  p.direct = aligned && a.stride_ks >= 0 && a.stride_vs >= 0 && a.stride_kb >= 0 && a.stride_vb >= 0 &&
             span < (int64_t(1) << 31) && block_bytes < (int64_t(1) << 32);
  p.nwg = with_config(a, p.C, [](auto cfg) {
    using K = decltype(cfg);
    return resident_groups<K::D, K::C, typename K::T, K::FP8>();
  });
  if (p.nwg <= 0) return false;
  const int64_t slots = 2 * static_cast<int64_t>(p.nwg);  // a share's first and last piece
  const int64_t rows_seg = p.rows_seg;
  // a segment's end, in quarter tiles: its rows' query loads and output stores (96 rows at D 256: 4.5 tiles' time,
  // measured at batch 64), the stores counted at 1.5 times their bytes; kept below seven tiles, so that no share's
  // cost span (at least 8 tiles) can fall between two tiles
  {
    const int64_t tile_bytes = static_cast<int64_t>(kTileKeys) * a.D * 2 * 2;
    const int64_t end_bytes = static_cast<int64_t>(p.rows_seg) * a.D * 2 * 2;
    const int64_t e = (4 * 3 * end_bytes + tile_bytes) / (2 * tile_bytes);
    p.seg_cost = p.fp8 ? 0 : static_cast<int>(e < 24 ? e : 24);  // fp8 tiles are compute-bound: not measured
  }
  // workspace: tiles before each request (int64 [B + 1]), the shares holding each segment's first and last tiles
  // (int32 [B HR][2]), partials, lse
  p.part_off = (2 * (static_cast<int64_t>(a.num_reqs) + 1) + 2 * static_cast<int64_t>(a.num_reqs) * p.HR + 63) / 64 * 64;
  p.lse_off = p.part_off + slots * rows_seg * a.D;
  return slots * rows_seg * a.D * 4 < (int64_t(1) << 30);  // partial rows addressed by 32-bit byte offsets
}

int64_t stream_workspace_bytes(const StreamPlan& p, const eagle4_attn_args&) {
  const int64_t slots = 2 * static_cast<int64_t>(p.nwg);
  return (p.lse_off + slots * p.rows_seg) * static_cast<int64_t>(sizeof(float));
}

int stream_launch(const eagle4_attn_args& a, const StreamPlan& p, hipStream_t s) {
  return with_config(a, p.C, [&](auto cfg) {
    using K = decltype(cfg);
    return launch<K::D, K::C, typename K::T, K::FP8>(a, p, s);
  });
}

}  // namespace e4attn
