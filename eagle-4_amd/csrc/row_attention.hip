// Attention of decode-time draft rows whose keys are mostly shared (kernels/row_attention.py), on gfx950.
//
// A request's rows see one range of its committed keys through its page table; the rows of a draft step (step > 0)
// all see the window frozen at the last committed position, [seq_len - window, seq_len - 1], plus their own `step`
// tree ancestors (KV slots), and extend rows (step == 0, row j at seq_len + j) see [pos - window + 1, pos] (:1-16).
//
// One workgroup per (key split, KV head and group of 64 rows, request): a row is (row of the request, query head of
// the KV head's group), so one read of each key serves all the rows of all G query heads (the reference's grid is per
// query head and reads every key G times). 32-key tiles of K and V go straight from HBM into a double-buffered LDS
// tile (global_load_lds, the verify attention's swizzled layout) one tile ahead, their slots looked up two tiles
// ahead; each wave runs the verify
// attention's tile step (S^T = K Q^T and O^T = V^T P^T on the 16x16x32 MFMA, online softmax in the log2 domain) for
// its 16 rows with a per-row key range. A draft step's ancestors are one more split. Every split leaves an fp32
// partial and its log2-sum-exp in the caller's scratch; a second kernel merges them (:213-240).

#include "attention_tile.h"

namespace {

using namespace e4attn;

constexpr int NW = 4;  // waves per workgroup: 64 rows
constexpr int NT = 64 * NW;

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
  __shared__ __attribute__((aligned(1024))) char smem[2][2][TL::BYTES];  // [buffer][K, V]

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
  // n = w + NW m. A lane's rows are looked up (page table or ancestor list) two tiles ahead, so the lookup's latency
  // hides behind a tile, and the tile's K / V load one tile ahead into the other LDS buffer.
  constexpr int RPI = TL::RPI, NI = TL::NI, NIW = NI / NW;
  static_assert(NI % NW == 0, "instructions per wave");
  uint32_t raw[NIW], rem[NIW];  // page-table entry and position within the page (or the ancestor's KV slot)
  auto lookup = [&](int tile) {
    const int64_t base = start + static_cast<int64_t>(tile) * kTileKeys;
#pragma unroll
    for (int i = 0; i < NIW; ++i) {
      const int row = (wave + NW * i) * RPI + lane / CH;
      const int64_t c = base + row < end ? base + row : end - 1;  // past the split: its last key (masked later)
      if (anc) {
        const int owner = static_cast<int>(c / a.max_depth), dep = static_cast<int>(c % a.max_depth);
        // owner < rows_per_request: the split ends at rows * max_depth. A column past the row's `step` ancestors
        // loads the row's first ancestor instead (written: the split exists only for step >= 1), so the masked key
        // multiplies finite data, never a slot nobody wrote
        const bool valid = dep < a.step;
        raw[i] = static_cast<uint32_t>(
            a.ancestors[(static_cast<int64_t>(b) * a.rows_per_request + owner) * a.max_depth + (valid ? dep : 0)]);
        rem[i] = 0;  // unused by the ancestor split; defined on both paths (left undefined, 12 registers spilled)
      } else {
        const uint32_t pos = static_cast<uint32_t>(c), tp = static_cast<uint32_t>(a.table_page);
        const uint32_t pg = tp_shift >= 0 ? pos >> tp_shift : pos / tp;
        raw[i] = static_cast<uint32_t>(table[pg]);
        rem[i] = pos - pg * tp;
      }
    }
  };
  auto issue = [&](int tile) {
    char* const kb = smem[tile & 1][0];
    char* const vb = smem[tile & 1][1];
#pragma unroll
    for (int i = 0; i < NIW; ++i) {
      const int n = wave + NW * i, row = n * RPI + lane / CH, pc = lane % CH;
      const uint32_t slot = anc ? raw[i] : raw[i] * static_cast<uint32_t>(a.table_page) + rem[i];
      const uint32_t cpg = static_cast<uint32_t>(a.cache_page);
      const uint32_t blk = cp_shift >= 0 ? slot >> cp_shift : slot / cpg, in = slot - blk * cpg;
      const int64_t koff = 2 * (blk * a.k_stride_page + in * a.k_stride_slot + kvh * a.k_stride_head);
      const int64_t voff = 2 * (blk * a.v_stride_page + in * a.v_stride_slot + kvh * a.v_stride_head + voff_packed);
      // the builtin takes its source as a plain pointer variable
      const char* ksrc = kc + koff + 16 * (pc ^ TL::kswz(row));
      const char* vsrc = vc + voff + 16 * (pc ^ TL::vswz(row));
      __builtin_amdgcn_global_load_lds(ksrc, kb + n * 1024, 16, 0, 2);
      __builtin_amdgcn_global_load_lds(vsrc, vb + n * 1024, 16, 0, 2);
    }
  };

  f32x4_t acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const float scale_log2 = a.scale * 1.4426950408889634f;
  const bool wave_rows = (grp * NW + wave) * 16 < R;  // a wave without rows loads, but skips the math
  if (ntiles > 0) {
    lookup(0);
    issue(0);
    if (ntiles > 1) lookup(1);
  }
  for (int x = 0; x < ntiles; ++x) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // tile x's loads (issued a tile ago) have landed, lookups too
    __syncthreads();  // ... for every wave, and the other buffer is no longer read
    if (x + 1 < ntiles) {
      issue(x + 1);
      if (x + 2 < ntiles) lookup(x + 2);
    }
    if (wave_rows) {
      const int64_t base = start + static_cast<int64_t>(x) * kTileKeys;
      tile_step_if<D, T>(smem[x & 1][0], smem[x & 1][1], qreg, acc, m, l, scale_log2, g, l16, [&](int k) {
        const int64_t c = base + k;
        if (!row_ok || c >= end) return false;
        const int64_t own = static_cast<int64_t>(t) * a.max_depth;  // a row's own ancestor columns
        if (anc) return c >= own && c < own + a.step;
        return c >= lo && c <= hi;
      });
    }
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
  float top = -INFINITY;
  for (int s = 0; s < splits; ++s) top = fmaxf(top, a.part_lse[part0 + s * a.rows_padded]);
  float wsum = 0.f;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
    const int64_t part = part0 + s * a.rows_padded;
    const float lse = a.part_lse[part];
    const float w = lse == -INFINITY ? 0.f : exp2f(lse - top);
    wsum += w;
    if (w != 0.f) acc += w * *reinterpret_cast<const f32x4_t*>(a.part_out + part * D + d);
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
