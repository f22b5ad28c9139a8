// The 32-key tile of tree-verify attention shared by its two schedules (split-context and streamed): the LDS layout
// of a K / V tile, the MFMA operand reads, and one online-softmax step of a wave's 16 query rows.
#pragma once

#include "common.h"

namespace e4attn {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));  // a 16-byte MFMA operand as a native vector
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

// Splits whose partials a merge thread loads at once (the split-schedule, fp32 and draft-row merges).
constexpr int kMergeGroup = 8;
constexpr int kTileKeys = 32;

template <typename T>
E4_DEV f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  if constexpr (T::code == EAGLE4_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
}

// The same on native-vector operands (arrays of them stay in registers without the struct copies HIP's uint4 brings).
template <typename T>
E4_DEV f32x4_t mfma16(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (T::code == EAGLE4_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
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

// 8 fp8-e4m3 values (OCP) as 16-bit dtype T, exactly (every e4m3 value is both a bf16 and an fp16 value): four
// v_cvt_scalef32_pk_* with scale 1.
template <typename T>
E4_DEV uint4 widen_fp8x8(uint2 raw) {
  if constexpr (T::code == EAGLE4_BF16) {
    return make_uint4(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw.x, 1.0f, false)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw.x, 1.0f, true)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw.y, 1.0f, false)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw.y, 1.0f, true)));
  } else {
    return make_uint4(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw.x, 1.0f, false)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw.x, 1.0f, true)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw.y, 1.0f, false)),
                      __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(raw.y, 1.0f, true)));
  }
}

// A context tile of fp8 K / V pages in LDS (streamed schedule): 64 keys, so that it fills the bytes of a 32-key
// 16-bit tile; rows of D bytes, 16-byte chunks XOR-swizzled in their low three index bits per row, so the consumers'
// 8-byte operand reads fall on distinct banks — K: 16 key rows at one d offset (chunk c of key k at c ^ (k & 7)); V,
// read transposed (ds_read_b64_tr_b8): 8 key rows, both halves of one chunk (chunk c of key k at
// c ^ ((k & 3) | (k >> 2 & 4))). Both swizzles repeat every 32 rows. Direct loads fill 1 KB runs as for 16-bit tiles.
constexpr int kTileKeys8 = 64;

template <int D>
struct Tile8 {
  static constexpr int CH = D / 16;          // 16-byte chunks per row
  static constexpr int ROWB = D;             // bytes per row
  static constexpr int BYTES = kTileKeys8 * ROWB;
  static constexpr int RPI = 1024 / ROWB;    // rows one direct-load instruction fills
  static constexpr int NI = kTileKeys8 / RPI;  // instructions per matrix per tile
  static constexpr int SW = CH < 8 ? CH - 1 : 7;
  static E4_DEV int kswz(int row) { return row & SW; }
  static E4_DEV int vswz(int row) { return ((row & 3) | ((row >> 2) & 4)) & SW; }
};

// A 32-key tile of K and of V lives in LDS row-major (rows of D 16-bit values) with its 16-byte chunks XOR-swizzled
// per row, so both MFMA operand reads are conflict-free on gfx950's LDS, which serves 256 bytes a cycle: 16 lanes of a
// 16-byte read (K: 16 consecutive key rows at one d offset) and 32 lanes of the transposing 8-byte read (V: 8 key rows,
// 32 bytes each) must fall in distinct 16- / 8-byte slots of a 256-byte window. With R = rows per 256 bytes (1 at
// D >= 128), K chunk c of key k sits at c ^ ((k / R) & (16 / R - 1)) and V chunk c at c ^ 2 ((k / R) & (8 / R - 1)).
// (Measured on the device, 4 waves per CU reading concurrently: a 3-bit K swizzle at D 256 took 34 cycles per read
// against 21 for this one and for linear addresses; the 2-bit V swizzle 20.5 against 18.) Direct loads
// (global_load_lds: lane p of an instruction fills 16-byte slot p of a 1 KB run) fetch for each slot the chunk the
// swizzle puts there.
template <int D>
struct Tile {
  static constexpr int CH = D / 8;           // 16-byte chunks per row
  static constexpr int ROWB = 2 * D;         // bytes per row
  static constexpr int BYTES = kTileKeys * ROWB;
  static constexpr int RPI = 1024 / ROWB;    // rows one direct-load instruction fills (64 lanes x 16 bytes)
  static constexpr int NI = kTileKeys / RPI;  // instructions per matrix per tile
  static constexpr int R = ROWB >= 256 ? 1 : 256 / ROWB;  // rows per 256-byte window
  static constexpr int KB = 4 / R;  // K chunk groups 4 c + g whose index bits the swizzle reaches (c % KB)
  static constexpr int VB = 8 / R;  // V d-tiles (chunk pairs 2 dt, 2 dt + 1) whose index bits it reaches (dt % VB)
  static constexpr E4_DEV int kswz(int row) { return (row / R) & (16 / R - 1); }
  static constexpr E4_DEV int vswz(int row) { return 2 * ((row / R) & (8 / R - 1)); }
};

// One tile for a wave's 16 query rows (lane l16 of each 16-lane group owns row l16; g = lane / 16):
//   S^T = K Q^T on v_mfma_f32_16x16x32 (s[kt][i] is key 16 kt + 4 g + i of the lane's row), masked — context keys
//   below `hi`, draft keys below `width` whose bit is set in the row's ancestor mask — then the online-softmax update
//   in the log2 domain (4 lanes share a row) and O^T = alpha O^T + V^T P^T, with P^T straight from registers as the
//   B operand and V^T read by transposing LDS loads (ds_read_b64_tr_b16) of the row-major tile.
// The reference's step is kernels/online_softmax.py:11-24 (max, rescale, exp, sum) over vllm/verify_attention.py
// :62-112's masked scores.
// tile_step_if takes the visibility as a predicate ok(key of the tile) of the lane's row.
template <int D, typename T, typename Ok>
E4_DEV void tile_step_if(const char* sKb, const char* sVb, const uint4 (&qreg)[D / 32], f32x4_t (&acc)[D / 16],
                         float& m, float& l, float scale_log2, int g, int l16, Ok ok);

template <int D, typename T>
E4_DEV void tile_step(const char* sKb, const char* sVb, const uint4 (&qreg)[D / 32], f32x4_t (&acc)[D / 16], float& m,
                      float& l, float scale_log2, bool is_new, int base, int hi, int width, int64_t row_mask, int g,
                      int l16) {
  tile_step_if<D, T>(sKb, sVb, qreg, acc, m, l, scale_log2, g, l16, [&](int k) {
    const int key = base + k;
    return is_new ? (key < width && ((row_mask >> key) & 1)) : key < hi;
  });
}

template <int D, typename T, typename Ok>
E4_DEV void tile_step_if(const char* sKb, const char* sVb, const uint4 (&qreg)[D / 32], f32x4_t (&acc)[D / 16],
                         float& m, float& l, float scale_log2, int g, int l16, Ok ok) {
  using TL = Tile<D>;
  f32x4_t s[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    const int key = 16 * kt + l16;
    const char* kr = sKb + key * TL::ROWB;
#pragma unroll
    for (int c = 0; c < D / 32; ++c)
      s[kt] = mfma16<T>(*reinterpret_cast<const uint4*>(kr + 16 * ((4 * c + g) ^ TL::kswz(key))), qreg[c], s[kt]);
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = ok(16 * kt + 4 * g + i) ? s[kt][i] * scale_log2 : -INFINITY;
      s[kt][i] = v;
      tmax = fmaxf(tmax, v);
    }
  }
  tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
  const float m_new = fmaxf(m, tmax);
  const float safe = m_new == -INFINITY ? 0.f : m_new;
  const float alpha = exp2f(m - safe);
  float psum = 0.f;
  uint32_t w[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {  // element i of P^T's operand is key 16 (i / 4) + 4 g + i % 4
    const float p0 = exp2f(s[p >> 1][2 * (p & 1)] - safe);
    const float p1 = exp2f(s[p >> 1][2 * (p & 1) + 1] - safe);
    psum += p0 + p1;
    w[p] = pack2<T>(p0, p1);
  }
  const uint4 pb = make_uint4(w[0], w[1], w[2], w[3]);
  psum += __shfl_xor(psum, 16, 64);
  psum += __shfl_xor(psum, 32, 64);
  l = l * alpha + psum;
  m = m_new;
  const int j = l16 >> 2, s4 = l16 & 3;
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    const int lc = 2 * dt + (s4 >> 1), half = 8 * (s4 & 1);
    const int k0 = 4 * g + j, k1 = 16 + 4 * g + j;
    const v4i16 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(sVb + k0 * TL::ROWB + 16 * (lc ^ TL::vswz(k0)) + half));
    const v4i16 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) v4i16*)(sVb + k1 * TL::ROWB + 16 * (lc ^ TL::vswz(k1)) + half));
    uint4 va;
    va.x = __builtin_bit_cast(uint2, lo4).x;
    va.y = __builtin_bit_cast(uint2, lo4).y;
    va.z = __builtin_bit_cast(uint2, hi4).x;
    va.w = __builtin_bit_cast(uint2, hi4).y;
    acc[dt] *= alpha;
    acc[dt] = mfma16<T>(va, pb, acc[dt]);
  }
}

// Loads a row's Q as the B operand of S^T = K Q^T: qreg[c] holds d = 32 c + 8 g + (0..7).
template <int D>
E4_DEV void load_q(uint4 (&qreg)[D / 32], const uint16_t* qrow, bool ok, int g) {
#pragma unroll
  for (int c = 0; c < D / 32; ++c)
    qreg[c] = ok ? *reinterpret_cast<const uint4*>(qrow + 32 * c + 8 * g) : make_uint4(0, 0, 0, 0);
}
template <int D>
E4_DEV void load_q(u32x4_t (&qreg)[D / 32], const uint16_t* qrow, bool ok, int g) {
#pragma unroll
  for (int c = 0; c < D / 32; ++c)
    qreg[c] = ok ? *reinterpret_cast<const u32x4_t*>(qrow + 32 * c + 8 * g) : u32x4_t{0u, 0u, 0u, 0u};
}

// The normalised output of a wave's rows: acc[dt][i] is d = 16 dt + 4 g + i.
template <int D, typename T>
E4_DEV void store_rows(uint16_t* orow, const f32x4_t (&acc)[D / 16], float inv, int g) {
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt)
    *reinterpret_cast<u32x2_t*>(orow + 16 * dt + 4 * g) =
        u32x2_t{pack2<T>(acc[dt][0] * inv, acc[dt][1] * inv), pack2<T>(acc[dt][2] * inv, acc[dt][3] * inv)};
}

// An fp32 partial (normalised by its own sum) of a wave's rows, for the merge.
template <int D>
E4_DEV void store_partial(float* prow, const f32x4_t (&acc)[D / 16], float inv, int g) {
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) *reinterpret_cast<f32x4_t*>(prow + 16 * dt + 4 * g) = acc[dt] * inv;
}

// ---- the streamed schedule (verify_attention_stream.hip) ------------------------------------------------------------
constexpr int kStreamMaxReqs = 1024;  // per-request query starts and contexts are kept in LDS

struct StreamPlan {
  int G, row_tiles, C, RG, HR, rows_seg, nwg, direct, fp8;
  int seg_cost;  // a segment's end in quarter tiles, for the cost-weighted shares
  int64_t part_off, lse_off;  // float offsets into the workspace (the int64 prefix of tiles per request is first)
};

// One request whose block table holds at most 4096 keys is too small for the streamed schedule's per-workgroup setup
// (~10 us of table loads, share search and ring fill before the first tile): the split schedule with 96-key splits
// finishes sooner (batch 1, L 512, D 128 bf16: 15.5 against 18.4 us; splits of 32 / 64 keys 19.3 / 16.3 us). A
// caller's own chunk is kept.
inline bool small_attention_job(const eagle4_attn_args& a) {
  return a.chunk <= 0 && a.num_reqs == 1 && static_cast<int64_t>(a.max_blocks) * a.page <= 4096;
}
constexpr int kSmallJobChunk = 96;

bool stream_covered(const eagle4_attn_args& a);
bool stream_plan(const eagle4_attn_args& a, StreamPlan& p);
int64_t stream_workspace_bytes(const StreamPlan& p, const eagle4_attn_args& a);
int stream_launch(const eagle4_attn_args& a, const StreamPlan& p, hipStream_t s);

// ---- fp32 rows over fp32 pages (verify_attention_f32.hip) ----------------------------------------------------------
bool f32_covered(const eagle4_attn_args& a);
int64_t f32_workspace_bytes(const eagle4_attn_args& a);
int f32_launch(const eagle4_attn_args& a, hipStream_t s);

}  // namespace e4attn
