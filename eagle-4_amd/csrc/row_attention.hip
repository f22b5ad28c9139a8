// Attention of decode-time draft rows whose keys are mostly shared (kernels/row_attention.py), on gfx950.
//
// A request's rows see one range of its committed keys through its page table; the rows of a draft step (step > 0)
// all see the window frozen at the last committed position, [seq_len - window, seq_len - 1], plus their own `step`
// tree ancestors (KV slots), and extend rows (step == 0, row j at seq_len + j) see [pos - window + 1, pos] (:1-16).
//
// One workgroup per (key split, KV head and group of 64 rows, request): a row is (row of the request, query head of
// the KV head's group), so one read of each key serves all the rows of all G query heads (the reference's grid is per
// query head and reads every key G times). 32-key tiles of K and V go straight from HBM into a three-stage LDS ring
// (global_load_lds, the verify attention's swizzled layout) two tiles ahead, their slots looked up (page-table entries
// or ancestor slots, also loaded straight into LDS) two tiles further ahead; with three workgroups per CU and, at a
// draft step's 16 rows per KV head, one wave of four computing, a double buffer one tile ahead held too few bytes in
// flight (3.9 TB/s). Each wave runs the verify attention's tile step (S^T = K Q^T and O^T = V^T P^T on the 16x16x32
// MFMA, online softmax in the log2 domain) for its 16 rows with a per-row key range. A draft step's ancestors are one more split. Every split leaves an fp32
// partial and its log2-sum-exp in the caller's scratch; a second kernel merges them (:213-240).

#include "attention_tile.h"

#pragma clang diagnostic ignored "-Winline-asm"  // the direct loads set M0; no compiler-generated code here uses M0

namespace {

using namespace e4attn;

constexpr int NW = 4;  // waves per workgroup: 64 rows
constexpr int NT = 64 * NW;
constexpr int kRing = 3;  // LDS stages of the streamed path

E4_DEV uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// 64 lanes x 16 bytes from per-lane global addresses into LDS [lds, lds + 1024), lane p at lds + 16 p, read once
// (nontemporal).
E4_DEV void dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(lds) : "memory", "m0");
}

template <int N>
E4_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// First key position a query at `pos` sees (window <= 0: the whole context) (:75-81).
E4_DEV int64_t window_start(int64_t pos, int window) {
  if (window <= 0) return 0;
  const int64_t s = pos - window + 1;
  return s > 0 ? s : 0;
}

template <int D, typename T>
__global__ __launch_bounds__(NT) void row_attention_kernel(const eagle4_row_attn_args a, int groups) {
  using TL = Tile<D>;
  constexpr int CH = D / 8;                      // 16-byte chunks per key row
  __shared__ __attribute__((aligned(1024))) char smem[kRing][2][TL::BYTES];  // [stage][K, V]

  const int split = blockIdx.x, kvh = blockIdx.y / groups, grp = blockIdx.y % groups, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, g = lane >> 4, l16 = lane & 15;
  const int G = a.heads / a.kv_heads, R = a.rows_per_request * G, NS = a.splits;
  const bool extend = a.step == 0;
  const int64_t seq_len = e4::ld(a.seq_lens, b);
  const int64_t trow = a.table_rows.ptr != nullptr ? e4::ld(a.table_rows, b) : b;
  const int32_t* const table = a.table + trow * a.stride_table;

  // this lane's row: request row t, query head `head`
  const int rho = (grp * NW + wave) * 16 + l16;
  const int t = rho / G, head = kvh * G + rho % G;
  const bool row_ok = rho < R;
  uint4 qreg[D / 32];
  const int64_t qrow = static_cast<int64_t>(b) * a.rows_per_request + t;
  const uint16_t* const qp = static_cast<const uint16_t*>(a.q) + qrow * a.stride_q_row;
  load_q<D>(qreg, qp + static_cast<int64_t>(head) * a.stride_q_head, row_ok, g);

  // the split's keys: positions [start, end) of the shared range, or (the last split of a draft step) the rows'
  // ancestor columns [0, rows * max_depth)
  const bool anc = !extend && split == NS;
  int64_t start = 0, end = 0, lo = 0, hi = -1;  // lo, hi: this row's own key range (positions)
  if (!anc) {
    int64_t first, last;
    if (extend) {
      first = window_start(seq_len, a.window);
      last = seq_len + a.rows_per_request - 1;
      lo = window_start(seq_len + t, a.window);
      hi = seq_len + t;
    } else {
      first = window_start(seq_len - 1, a.window);
      last = seq_len - 1;
      lo = first;
      hi = last;
    }
    const int64_t span = last + 1 - first;
    const int64_t per = span > 0 ? ((span + NS - 1) / NS + kTileKeys - 1) / kTileKeys * kTileKeys : 0;
    start = first + split * per;
    end = start + per < last + 1 ? start + per : last + 1;
  } else {
    end = static_cast<int64_t>(a.rows_per_request) * a.max_depth;
  }
  const int ntiles = end > start ? static_cast<int>((end - start + kTileKeys - 1) / kTileKeys) : 0;

  // element offsets of a key's K and V rows in the caches: key k of the tile starting at `base`
  const char* const kc = static_cast<const char*>(a.keys);
  const char* const vc = static_cast<const char*>(a.values != nullptr ? a.values : a.keys);
  const int64_t voff_packed = a.values != nullptr ? 0 : D;  // packed [K, V] rows: V follows K
  // page sizes as shifts when they are powers of two (the common case; a division otherwise)
  const int tp_shift = (a.table_page & (a.table_page - 1)) == 0 ? __builtin_ctz(a.table_page) : -1;
  const int cp_shift = (a.cache_page & (a.cache_page - 1)) == 0 ? __builtin_ctz(a.cache_page) : -1;
  // Direct loads (global_load_lds): instruction n of a tile fills 1 KB run n of the LDS tile, lane p its 16-byte slot
  // p — row n * RPI + p / CH, the chunk the tile's swizzle puts at slot p % CH. Wave w issues instructions
  // n = w + NW i. Per tile a wave issues one lookup — lane j < NIW RPI loads the page-table entry (or the ancestor's
  // KV slot) of row j of its instructions straight into LDS — and, two tiles later, its K and V loads from per-lane
  // addresses built from those entries; the loads run two tiles ahead of the compute through a three-stage ring.
  // Lookups and loads are issued from inline assembly and waited for by count (vector memory operations retire in
  // issue order): the compiler, which would wait for every load before the tile step's first LDS read, sees neither.
  constexpr int RPI = TL::RPI, NI = TL::NI, NIW = NI / NW;
  static_assert(NI % NW == 0 && NIW * RPI <= 64, "instructions per wave");
  __shared__ int32_t s_ent[4][NW][64];  // a ring of four tiles' lookups per wave
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  auto key_of = [&](int tile, int row) {  // the key a tile row loads: past the split, the split's last key (masked)
    const int64_t c = start + static_cast<int64_t>(tile) * kTileKeys + row;
    return c < end ? c : end - 1;
  };
  auto lookup = [&](int tile) {
    const int j = lane < NIW * RPI ? lane : 0;
    const int64_t c = key_of(tile, (wv + NW * (j / RPI)) * RPI + j % RPI);
    const int32_t* src;
    if (anc) {
      // owner < rows_per_request: the split ends at rows * max_depth. A column past the row's `step` ancestors
      // loads the row's first ancestor instead (written: the split exists only for step >= 1), so the masked key
      // multiplies finite data, never a slot nobody wrote
      const int ci = static_cast<int>(c), owner = ci / a.max_depth, dep = ci - owner * a.max_depth;
      src = a.ancestors + (static_cast<int64_t>(b) * a.rows_per_request + owner) * a.max_depth + (dep < a.step ? dep : 0);
    } else {
      const uint32_t pos = static_cast<uint32_t>(c), tp = static_cast<uint32_t>(a.table_page);
      src = table + (tp_shift >= 0 ? pos >> tp_shift : pos / tp);
    }
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src),
                 "s"(lds_addr(&s_ent[tile & 3][wv][0])) : "memory", "m0");
  };
  auto issue = [&](int tile, int stage) {
    const uint32_t kl = lds_addr(smem[stage][0]), vl = lds_addr(smem[stage][1]);
#pragma unroll
    for (int i = 0; i < NIW; ++i) {
      const int n = wv + NW * i, row = n * RPI + lane / CH, pc = lane % CH;
      const uint32_t ent = static_cast<uint32_t>(s_ent[tile & 3][wv][i * RPI + lane / CH]);
      uint32_t slot = ent;
      if (!anc) {
        const uint32_t pos = static_cast<uint32_t>(key_of(tile, row)), tp = static_cast<uint32_t>(a.table_page);
        const uint32_t pg = tp_shift >= 0 ? pos >> tp_shift : pos / tp;
        slot = ent * tp + (pos - pg * tp);
      }
      const uint32_t cpg = static_cast<uint32_t>(a.cache_page);
      const uint32_t blk = cp_shift >= 0 ? slot >> cp_shift : slot / cpg, in = slot - blk * cpg;
      const int64_t koff = 2 * (blk * a.k_stride_page + in * a.k_stride_slot + kvh * a.k_stride_head);
      const int64_t voff = 2 * (blk * a.v_stride_page + in * a.v_stride_slot + kvh * a.v_stride_head + voff_packed);
      dma16(kc + koff + 16 * (pc ^ TL::kswz(row)), kl + n * 1024);
      dma16(vc + voff + 16 * (pc ^ TL::vswz(row)), vl + n * 1024);
    }
  };

  f32x4_t acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float scale_log2 = a.scale * 1.4426950408889634f;
  const bool wave_rows = (grp * NW + wave) * 16 < R;  // a wave without rows loads, but skips the math
  // prologue: the lookups of tiles 0 .. 3, then the loads of tiles 0 and 1
  constexpr int TL2 = 2 * NIW;  // loads per tile and wave
#pragma unroll
  for (int x = 0; x < 4; ++x)
    if (x < ntiles) lookup(x);
  // the lookups, and q: a wait the compiler sees, so that it places none of its own for q inside the loop (there it
  // would drain the ring)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  if (ntiles > 0) issue(0, 0);
  if (ntiles > 1) issue(1, 1);
  int stage = 0;
  for (int x = 0; x < ntiles; ++x) {
    // Issued after tile x's loads: the lookup of x + 2 (from x = 2; before, the prologue's, already waited for),
    // then the loads of x + 1 and the lookup of x + 3 (from x = 1). Waiting until only the last two groups are
    // outstanding lands tile x's loads and the lookup of x + 2.
    const int newer = (x + 1 < ntiles ? TL2 : 0) + (x >= 1 && x + 3 < ntiles ? 1 : 0);
    if (newer == TL2 + 1)
      wait_vm<TL2 + 1>();
    else if (newer == TL2)
      wait_vm<TL2>();
    else if (newer == 1)
      wait_vm<1>();
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // ... for every wave, and stage x - 1 is no longer read
    if (x + 2 < ntiles) {
      issue(x + 2, stage == 0 ? kRing - 1 : stage - 1);
      if (x + 4 < ntiles) lookup(x + 4);
    }
    if (wave_rows) {
      const int64_t base = start + static_cast<int64_t>(x) * kTileKeys;
      tile_step_if<D, T>(smem[stage][0], smem[stage][1], qreg, acc, m, l, scale_log2, g, l16, [&](int k) {
        const int64_t c = base + k;
        if (!row_ok || c >= end) return false;
        const int64_t own = static_cast<int64_t>(t) * a.max_depth;  // a row's own ancestor columns
        if (anc) return c >= own && c < own + a.step;
        return c >= lo && c <= hi;
      });
    }
    stage = stage == kRing - 1 ? 0 : stage + 1;
  }

  // the split's partial of this row (:186-199): out / denominator and the log2-sum-exp
  if (row_ok) {
    const int64_t part = ((static_cast<int64_t>(b) * a.heads + head) * (NS + 1) + split) * a.rows_padded + t;
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    store_partial<D>(a.part_out + part * D, acc, inv, g);
    if (g == 0) a.part_lse[part] = l > 0.f ? m + log2f(l) : -INFINITY;
  }
}

// _merge_splits_kernel (:202-224): D / 4 lanes per (row, query head), 4 consecutive columns each (16-byte loads of
// the partials), 256 / (D / 4) pairs per workgroup; weights 2^(lse - max) over the splits.
template <int D, typename T>
__global__ __launch_bounds__(256) void row_merge_kernel(const eagle4_row_attn_args a, int splits) {
  constexpr int LP = D / 4, PAIRS = 256 / LP;
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * PAIRS + threadIdx.x / LP;
  const int d = 4 * (threadIdx.x % LP);
  if (pair >= static_cast<int64_t>(a.bs) * a.rows_per_request * a.heads) return;
  const int64_t row = pair / a.heads;
  const int head = static_cast<int>(pair % a.heads);
  const int64_t b = row / a.rows_per_request, t = row % a.rows_per_request;
  const int64_t part0 = ((b * a.heads + head) * (a.splits + 1)) * a.rows_padded + t;
  // The splits in groups of kMergeGroup, every load of a group issued before the first is used (one memory round trip
  // per group, not per split; a group's loads past the last split re-read the first), the same operations in the same
  // order as one split at a time.
  float top = -INFINITY;
  for (int s0 = 0; s0 < splits; s0 += kMergeGroup) {
    float l[kMergeGroup];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i) l[i] = a.part_lse[part0 + (s0 + i < splits ? s0 + i : s0) * a.rows_padded];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i)
      if (s0 + i < splits) top = fmaxf(top, l[i]);
  }
  float wsum = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += kMergeGroup) {
    float l[kMergeGroup];
    f32x4_t v[kMergeGroup];
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i) {
      const int64_t part = part0 + (s0 + i < splits ? s0 + i : s0) * a.rows_padded;
      l[i] = a.part_lse[part];
      v[i] = *reinterpret_cast<const f32x4_t*>(a.part_out + part * D + d);
    }
#pragma unroll
    for (int i = 0; i < kMergeGroup; ++i) {
      if (s0 + i >= splits) break;
      const float w = l[i] == -INFINITY ? 0.f : exp2f(l[i] - top);
      wsum += w;
      if (w != 0.f) acc += w * v[i];
    }
  }
  uint16_t* o = static_cast<uint16_t*>(a.out) + row * a.stride_o_row + static_cast<int64_t>(head) * a.stride_o_head + d;
  const uint32_t lo = T::from_f32(acc.x / wsum) | (static_cast<uint32_t>(T::from_f32(acc.y / wsum)) << 16);
  const uint32_t hi = T::from_f32(acc.z / wsum) | (static_cast<uint32_t>(T::from_f32(acc.w / wsum)) << 16);
  *reinterpret_cast<uint2*>(o) = make_uint2(lo, hi);
}

template <int D, typename T>
int launch(const eagle4_row_attn_args& a, hipStream_t s) {
  const int R = a.rows_per_request * (a.heads / a.kv_heads);
  const int groups = (R + 16 * NW - 1) / (16 * NW);
  const int splits = a.splits + (a.step == 0 ? 0 : 1);
  row_attention_kernel<D, T><<<dim3(splits, a.kv_heads * groups, a.bs), NT, 0, s>>>(a, groups);
  const int64_t pairs = static_cast<int64_t>(a.bs) * a.rows_per_request * a.heads, per = 256 / (D / 4);
  row_merge_kernel<D, T><<<static_cast<unsigned>((pairs + per - 1) / per), 256, 0, s>>>(a, splits);
  return E4_LAUNCH_STATUS();
}

template <typename T>
int launch_d(const eagle4_row_attn_args& a, hipStream_t s) {
  switch (a.head_dim) {
    case 64: return launch<64, T>(a, s);
    case 128: return launch<128, T>(a, s);
    case 256: return launch<256, T>(a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}

}  // namespace

extern "C" int eagle4_row_attention(const eagle4_row_attn_args* a, void* stream) {
  if (a->bs == 0 || a->rows_per_request == 0) return EAGLE4_OK;
  const auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (a->kv_heads <= 0 || a->heads % a->kv_heads || a->splits < 1 || a->bs > 65535 || a->step < 0 ||
      a->rows_per_request < 1 || a->rows_padded < a->rows_per_request || a->table == nullptr ||
      a->seq_lens.ptr == nullptr || a->table_page < 1 || a->cache_page < 1 ||
      (a->step > 0 && (a->ancestors == nullptr || a->max_depth < a->step)) ||
      (a->dtype != EAGLE4_BF16 && a->dtype != EAGLE4_F16) || !al16(a->q) || !al16(a->keys) ||
      (a->values != nullptr && !al16(a->values)) || a->stride_q_row % 8 || a->stride_q_head % 8 ||
      a->k_stride_page % 8 || a->k_stride_slot % 8 || a->k_stride_head % 8 || a->v_stride_page % 8 ||
      a->v_stride_slot % 8 || a->v_stride_head % 8 || reinterpret_cast<uintptr_t>(a->out) % 8 ||
      a->stride_o_row % 4 || a->stride_o_head % 4 ||
      a->part_rows < static_cast<int64_t>(a->bs) * a->heads * (a->splits + 1) * a->rows_padded)
    return EAGLE4_NOT_COVERED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  return a->dtype == EAGLE4_BF16 ? launch_d<e4::Bf16>(*a, s) : launch_d<e4::F16>(*a, s);
}
