// Gated delta rule over a draft tree on gfx950, snapshot contract (kernels/gdn_tree_recurrence.py:204-359, 562-706).
//
// Roofline: HBM writes. Every node of every (request, value head) writes its whole fp32 [V, K] state (64 KB at
// V = K = 128) and reads ~1 KB of inputs, at ~1.7 FLOP per byte. The layout is chosen for the stores:
//
//  * A workgroup owns one (V tile, request, value head) and walks the request's nodes in order; the state tile lives
//    in VGPRs for the whole walk.
//  * C adjacent lanes share a V row, each holding E = K / C state values as E/4 float4 chunks at
//    k = 4c + 4Cj (c = lane % C, j = chunk). At K = 128, C = 8: one store instruction of a wave writes 8 rows x 128
//    contiguous bytes -> every snapshot store is full 128-byte lines, streamed once.
//  * The K reductions (h k and h q) are C-lane butterflies; q / k norms reduce the same way. No LDS is used.
//  * A chain child of an fp32 state continues from the registers (bitwise what a reload gives); any other node
//    reloads its parent's snapshot, which the same thread wrote (same addresses, same lane), so no barrier is needed.
//
// The math and its order follow the walk: h *= exp(g); v' = (v - h k) * beta; h += k v'; o = h q, with beta
// rounded through b's dtype and q, k L2-normalised with 1e-6 inside the square root.

#include "common.h"

namespace {

template <typename T>
E4_DEV void load4(const typename T::storage* p, float* out) {
  if constexpr (sizeof(typename T::storage) == 4) {
    const float4 v = *reinterpret_cast<const float4*>(p);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    out[0] = T::to_f32(static_cast<uint16_t>(v.x & 0xffffu));
    out[1] = T::to_f32(static_cast<uint16_t>(v.x >> 16));
    out[2] = T::to_f32(static_cast<uint16_t>(v.y & 0xffffu));
    out[3] = T::to_f32(static_cast<uint16_t>(v.y >> 16));
  }
}

template <typename T>
E4_DEV void store4(typename T::storage* p, const float* in) {
  if constexpr (sizeof(typename T::storage) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(in[0], in[1], in[2], in[3]);
  } else {
    uint2 v;
    v.x = static_cast<uint32_t>(T::from_f32(in[0])) | (static_cast<uint32_t>(T::from_f32(in[1])) << 16);
    v.y = static_cast<uint32_t>(T::from_f32(in[2])) | (static_cast<uint32_t>(T::from_f32(in[3])) << 16);
    *reinterpret_cast<uint2*>(p) = v;
  }
}

// A chunk of four state values of a runtime dtype (the initial-state pool may differ from the snapshot buffer).
E4_DEV void load4_code(const void* base, int64_t off, int dtype, float* out) {
  if (dtype == EAGLE4_F32)
    load4<e4::F32>(static_cast<const float*>(base) + off, out);
  else if (dtype == EAGLE4_BF16)
    load4<e4::Bf16>(static_cast<const uint16_t*>(base) + off, out);
  else
    load4<e4::F16>(static_cast<const uint16_t*>(base) + off, out);
}

// Per-node inputs of one lane: its E values of q and k, and v of its RPT rows.
template <int E, int RPT>
struct NodeIn {
  float q[E], k[E], v[RPT];
  float a, b;
  int32_t parent;
};

template <int K, int C, int RPT, typename Tin>
E4_DEV void load_node(NodeIn<K / C, RPT>& in, const eagle4_gdn_args& a, int64_t t, int n, int step, int ih, int hv,
                      int c, const int* rows, bool valid) {
  constexpr int E = K / C;
  using S = typename Tin::storage;
  if (!valid) return;
  const S* q = static_cast<const S*>(a.q) + t * a.stride_q + static_cast<int64_t>(ih) * K;
  const S* k = static_cast<const S*>(a.k) + t * a.stride_k + static_cast<int64_t>(ih) * K;
#pragma unroll
  for (int j = 0; j < E / 4; ++j) {
    load4<Tin>(q + 4 * c + 4 * C * j, &in.q[4 * j]);
    load4<Tin>(k + 4 * c + 4 * C * j, &in.k[4 * j]);
  }
  const S* v = static_cast<const S*>(a.v) + t * a.stride_v + static_cast<int64_t>(hv) * a.V;
#pragma unroll
  for (int s = 0; s < RPT; ++s) in.v[s] = rows[s] < a.V ? Tin::to_f32(v[rows[s]]) : 0.f;
  in.a = e4::load_scalar(a.a, t * a.stride_a + hv, a.gate_dtype);
  in.b = e4::load_scalar(a.b, t * a.stride_b + hv, a.gate_dtype);
  in.parent = static_cast<int32_t>(e4::ld(a.parents, n, step));
}

// One workgroup: 4 waves; rows of the V tile: RPT slots x 4 waves x (64 / C) rows.
template <int K, int C, int RPT, typename Tin, typename Tsnap>
__global__ __launch_bounds__(256) void gdn_tree_walk_kernel(const eagle4_gdn_args a) {
  constexpr int E = K / C;
  constexpr int NJ = E / 4;
  constexpr int ROWS_WAVE = 64 / C;
  constexpr int ROWS_WG = RPT * 4 * ROWS_WAVE;
  static_assert(E % 4 == 0 && C <= 64, "lane layout");
  using SS = typename Tsnap::storage;

  const int n = blockIdx.y, hv = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane % C, rr = lane / C;
  const int ih = hv / (a.HV / a.H);
  int rows[RPT];
#pragma unroll
  for (int s = 0; s < RPT; ++s) rows[s] = blockIdx.x * ROWS_WG + s * 4 * ROWS_WAVE + wave * ROWS_WAVE + rr;

  if (a.publish != nullptr && blockIdx.x == 0 && hv == 0) {  // _publish_slot_table (:188-200)
    for (int i = tid; i < a.num_slot_cols; i += blockDim.x)
      a.publish[n * a.stride_publish + i] = static_cast<int32_t>(e4::ld(a.snap_indices, n, i));
  }
  const int64_t bos = e4::ld(a.cu_seqlens, n);
  const int T = static_cast<int>(e4::ld(a.cu_seqlens, n + 1) - bos);

  // the initial state (:284-296); with num_accepted its slot is in column num_accepted - 1
  float h[RPT][E];
  int64_t idx = a.num_accepted.ptr != nullptr ? e4::ld(a.h0_indices, n, e4::ld(a.num_accepted, n) - 1)
                                              : e4::ld(a.h0_indices, n, 0);
  const int64_t head_off = static_cast<int64_t>(hv) * a.V * K;
#pragma unroll
  for (int s = 0; s < RPT; ++s) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (idx > a.pad_slot_id && rows[s] < a.V) {
        load4_code(a.h0_source, idx * a.stride_h0_source + head_off + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j,
                   a.h0_dtype, &h[s][4 * j]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) h[s][4 * j + e] = 0.f;
      }
    }
  }
  const int64_t cache_idx = e4::ld(a.snap_indices, n, 0);  // the request's scratch row (per-row slots: row 0's slot)
  const float A = -expf(e4::load_scalar(a.A_log, hv, a.A_log_dtype));
  const float dt_bias = e4::load_scalar(a.dt_bias, hv, a.dt_bias_dtype);
  SS* snap = static_cast<SS*>(a.snap);

  NodeIn<E, RPT> cur, nxt;
  load_node<K, C, RPT, Tin>(cur, a, bos, n, 0, ih, hv, c, rows, T > 0);
  for (int step = 0; step < T; ++step) {
    const int parent = cur.parent;
    load_node<K, C, RPT, Tin>(nxt, a, bos + step + 1, n, step + 1, ih, hv, c, rows, step + 1 < T);
    int64_t slot = cache_idx, parent_slot = cache_idx;
    if (a.row_slots) {
      slot = e4::ld(a.snap_indices, n, step);
      parent_slot = step != 0 ? e4::ld(a.snap_indices, n, parent) : a.pad_slot_id;  // the root reads nothing
    }
    bool reload = step != 0 && parent_slot > a.pad_slot_id;  // :318-329
    if (a.skip_chain_reload) reload = reload && parent != step - 1;
    if (reload) {
      const SS* src = snap + parent_slot * a.stride_snap_slot + static_cast<int64_t>(parent) * a.stride_snap_row + head_off;
#pragma unroll
      for (int s = 0; s < RPT; ++s)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          if (rows[s] < a.V) load4<Tsnap>(src + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j, &h[s][4 * j]);
    }
    // gate and write strength (:115-140)
    const float x = cur.a + dt_bias;
    const float bx = a.softplus_beta * x;
    const float softplus = bx <= a.softplus_threshold ? (1.0f / a.softplus_beta) * logf(1.0f + expf(bx)) : x;
    const float decay = expf(A * softplus);
    const float beta = e4::round_code(1.0f / (1.0f + expf(-cur.b)), a.gate_dtype);
    // L2 norms over K (:143-151)
    float qq = 0.f, kk = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      qq = fmaf(cur.q[e], cur.q[e], qq);
      kk = fmaf(cur.k[e], cur.k[e], kk);
    }
    qq = e4::group_sum<C>(qq);
    kk = e4::group_sum<C>(kk);
    const float qinv = 1.0f / sqrtf(qq + 1e-6f);
    const float kinv = 1.0f / sqrtf(kk + 1e-6f);
    float qn[E], kn[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      qn[e] = (cur.q[e] * qinv) * a.scale;
      kn[e] = cur.k[e] * kinv;
    }
    // the delta rule step (:167-185)
    float o[RPT];
#pragma unroll
    for (int s = 0; s < RPT; ++s) {
      float hk = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        h[s][e] *= decay;
        hk = fmaf(h[s][e], kn[e], hk);
      }
      hk = e4::group_sum<C>(hk);
      const float dv = (cur.v[s] - hk) * beta;
      float hq = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        h[s][e] = fmaf(kn[e], dv, h[s][e]);
        hq = fmaf(h[s][e], qn[e], hq);
      }
      o[s] = e4::group_sum<C>(hq);
    }
    const int64_t t = bos + step;
    if (c == 0) {
#pragma unroll
      for (int s = 0; s < RPT; ++s)
        if (rows[s] < a.V) e4::store_scalar(a.out, t * a.stride_o + static_cast<int64_t>(hv) * a.V + rows[s], a.out_dtype, o[s]);
    }
    if (slot > a.pad_slot_id) {
      SS* dst = snap + slot * a.stride_snap_slot + static_cast<int64_t>(step) * a.stride_snap_row + head_off;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int s = 0; s < RPT; ++s)
          if (rows[s] < a.V) store4<Tsnap>(dst + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j, &h[s][4 * j]);
    }
    cur = nxt;
  }
}

template <int K, int C, int RPT, typename Tin>
int launch_snap(const eagle4_gdn_args& a, hipStream_t s) {
  constexpr int ROWS_WG = RPT * 4 * (64 / C);
  const dim3 grid(e4::ceil_div(a.V, ROWS_WG), a.N, a.HV);
  if (a.snap_dtype == EAGLE4_F32)
    gdn_tree_walk_kernel<K, C, RPT, Tin, e4::F32><<<grid, 256, 0, s>>>(a);
  else if (a.snap_dtype == EAGLE4_BF16)
    gdn_tree_walk_kernel<K, C, RPT, Tin, e4::Bf16><<<grid, 256, 0, s>>>(a);
  else if (a.snap_dtype == EAGLE4_F16)
    gdn_tree_walk_kernel<K, C, RPT, Tin, e4::F16><<<grid, 256, 0, s>>>(a);
  else
    return EAGLE4_NOT_COVERED;
  return E4_LAUNCH_STATUS();
}

template <int K, int C, int RPT>
int launch_in(const eagle4_gdn_args& a, hipStream_t s) {
  if (a.in_dtype == EAGLE4_BF16) return launch_snap<K, C, RPT, e4::Bf16>(a, s);
  if (a.in_dtype == EAGLE4_F16) return launch_snap<K, C, RPT, e4::F16>(a, s);
  if (a.in_dtype == EAGLE4_F32) return launch_snap<K, C, RPT, e4::F32>(a, s);
  return EAGLE4_NOT_COVERED;
}

}  // namespace

extern "C" int eagle4_gdn_tree_recurrent_update(const eagle4_gdn_args* a, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->N == 0) return EAGLE4_OK;
  if (a->H <= 0 || a->HV % a->H != 0 || a->V <= 0 || !e4::is_float_dtype(a->gate_dtype) ||
      !e4::is_float_dtype(a->out_dtype) || !e4::is_float_dtype(a->h0_dtype) || a->snap_indices.ptr == nullptr ||
      a->parents.ptr == nullptr || a->cu_seqlens.ptr == nullptr || a->h0_indices.ptr == nullptr)
    return EAGLE4_NOT_COVERED;
  switch (a->K) {
    case 8: return launch_in<8, 2, 1>(*a, s);
    case 16: return launch_in<16, 4, 1>(*a, s);
    case 32: return launch_in<32, 8, 1>(*a, s);
    case 64: return launch_in<64, 8, 2>(*a, s);
    case 128: return launch_in<128, 8, 4>(*a, s);
    case 256: return launch_in<256, 8, 2>(*a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}
