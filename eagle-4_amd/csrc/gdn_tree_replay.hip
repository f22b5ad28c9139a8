// GDN records contract, rounded path replay on gfx950 (kernels/gdn_tree_records.py:16-101 with ROUND_STATE): every
// node of a request's tree steps from its parent's state rounded to the pool dtype (the root from the pool state),
// writes its output and its record (delta, normalised key, decay), and hands its own rounded state to its children.
//
// Since a child reads only its parent's ROUNDED state h~_p, everything a node writes follows from matrix products with
// 16-bit operands that are exact in the pool dtype: for a child j of p (decay e_j, beta_j, raw k_j, q_j, norm scales
// ks_j = 1 / |k_j|, qs_j = scale / |q_j|)
//   h~_p k^_j = ks_j (h~_p k_j),   delta_j = (v_j - e_j ks_j (h~_p k_j)) beta_j,
//   o_j = h_j q^_j = e_j qs_j (h~_p q_j) + delta_j ks_j qs_j (k_j . q_j),
// so all children of p are served by one MFMA pass over h~_p with [k_j | q_j] as the other operand (products exact,
// fp32 sums). Only a node with children needs its own state, h~_j = round(e_j h~_p + k^_j delta_j^T): a fused
// multiply-add per element and the hardware's packed round-to-nearest-even conversion. Leaves cost no state work.
//
// One wave owns 16 V rows of one (request, value head); a workgroup of four waves shares the request's staged node
// inputs in LDS. The state lives in registers as the MFMA's 16-bit operand (lane: row r16, K elements
// [g K / 4, (g + 1) K / 4) in blocks of 8). The wave walks the tree's internal nodes depth first: a node whose several
// children have children of their own parks its rounded state in a small register stack (the oldest entry is dropped
// when it is full); a parent whose entry was dropped is recomputed from the pool state along its root path with the
// deltas already in LDS. Deltas and output terms gather in LDS and leave at the end as 16- and 8-byte row runs. A
// request without records (record_indices < 0) runs its rows as one chain with an fp32 state and no rounding
// (:51-53).

#include "gdn_walk.h"

namespace e4replay {
int launch(const eagle4_records_args& a, hipStream_t s) __attribute__((visibility("hidden")));
}

namespace {

using namespace e4walk;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int WAVES = 4;          // waves per workgroup
constexpr int NT = 64 * WAVES;    // threads per workgroup
constexpr int ROWS = 16 * WAVES;  // V rows per workgroup

// The pool dtype's arithmetic: the MFMA over raw 16-bit operands, widening of the low / high element of a word, and
// the packed fp32 -> 16-bit conversion (round to nearest even: what a store to the pool dtype and a reload give).
template <typename T>
struct Ops;
template <>
struct Ops<e4::Bf16> {
  static E4_DEV f32x4_t mma(u32x4 x, u32x4 y, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, x), __builtin_bit_cast(bf16x8_t, y),
                                                   c, 0, 0, 0);
  }
  static E4_DEV float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static E4_DEV float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static E4_DEV uint32_t pack(float x0, float x1) {
    const f32x2_t v = {x0, x1};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  }
  static E4_DEV uint16_t narrow(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }
};
template <>
struct Ops<e4::F16> {
  static E4_DEV f32x4_t mma(u32x4 x, u32x4 y, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, x), __builtin_bit_cast(f16x8_t, y), c,
                                                  0, 0, 0);
  }
  static E4_DEV float lo(uint32_t w) { return e4::f16_to_f32(static_cast<uint16_t>(w & 0xffffu)); }
  static E4_DEV float hi(uint32_t w) { return e4::f16_to_f32(static_cast<uint16_t>(w >> 16)); }
  static E4_DEV uint32_t pack(float x0, float x1) {
    const f32x2_t v = {x0, x1};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
  }
  static E4_DEV uint16_t narrow(float x) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x)); }
};


// Keeps the compiler from moving LDS accesses across this point (a lane reads what other lanes of its wave wrote
// just before; LDS executes one wave's accesses in order).
E4_DEV void lds_order() { __asm__ volatile("" ::: "memory"); }

// ---- a request without records: one chain over its rows, fp32 state, no rounding (:51-53, :77-92) ------------------
// A rare path, kept small in registers so it does not cost the tree walk occupancy: the wave's 16 rows in two halves
// of 8, lane (g8, r8) holding row r8 of the half and K elements [g8 K / 8, (g8 + 1) K / 8), the raw q / k words
// widened where they are used.
template <int K, typename T>
E4_DEV void chain_walk(const eagle4_records_args& a, int64_t bos, int Tn, int idx, int hv, int ih, int row16,
                       int lane, float A, float dt_bias) {
  using O = Ops<T>;
  constexpr int EL = K / 8, CH = EL / 4;  // elements per lane, in 8-byte chunks
  const int r8 = lane & 7, g8 = lane >> 3;
  auto reduce = [](float x) {
    x += __shfl_xor(x, 8);
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
  };
  for (int half = 0; half < 2; ++half) {
    const int row = row16 + 8 * half + r8;
    float h[EL];
    {
      const uint16_t* sp = static_cast<const uint16_t*>(a.state) + (idx >= 0 ? idx : 0) * a.stride_state +
                           (static_cast<int64_t>(hv) * a.V + row) * K + g8 * EL;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const u32x2 raw = idx >= 0 ? *reinterpret_cast<const u32x2*>(sp + 4 * c) : u32x2{0u, 0u};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          h[4 * c + 2 * e] = O::lo(raw[e]);
          h[4 * c + 2 * e + 1] = O::hi(raw[e]);
        }
      }
    }
    for (int t = 0; t < Tn; ++t) {
      const int64_t tok = bos + t;
      const int64_t head = static_cast<int64_t>(ih) * K + g8 * EL;
      const uint16_t* kp = static_cast<const uint16_t*>(a.k) + tok * a.stride_k + head;
      const uint16_t* qp = static_cast<const uint16_t*>(a.q) + tok * a.stride_q + head;
      u32x2 kr[CH], qr[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        kr[c] = *reinterpret_cast<const u32x2*>(kp + 4 * c);
        qr[c] = *reinterpret_cast<const u32x2*>(qp + 4 * c);
      }
      const uint16_t vraw = static_cast<const uint16_t*>(a.v)[tok * a.stride_v + static_cast<int64_t>(hv) * a.V + row];
      const uint32_t ga = load_raw(a.a, tok * a.stride_a + hv, a.gate_dtype);
      const uint32_t gb = load_raw(a.b, tok * a.stride_b + hv, a.gate_dtype);
      float kk = 0.f, qq = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float k0 = O::lo(kr[c][e]), k1 = O::hi(kr[c][e]), q0 = O::lo(qr[c][e]), q1 = O::hi(qr[c][e]);
          kk = fmaf(k0, k0, fmaf(k1, k1, kk));
          qq = fmaf(q0, q0, fmaf(q1, q1, qq));
        }
      const float ks = 1.0f / sqrtf(reduce(kk) + 1e-6f), qs = a.scale / sqrtf(reduce(qq) + 1e-6f);  // (:147-150)
      const float2 gt = gate_of(ga, gb, a.gate_dtype, 1.0f, 20.0f, A, dt_bias);
      float hk = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float& h0 = h[4 * c + 2 * e];
          float& h1 = h[4 * c + 2 * e + 1];
          h0 *= gt.x;
          h1 *= gt.x;
          hk = fmaf(h0, O::lo(kr[c][e]), fmaf(h1, O::hi(kr[c][e]), hk));
        }
      const float dv = (O::lo(vraw) - reduce(hk) * ks) * gt.y;
      const float kd = dv * ks;
      float hq = 0.f;
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float& h0 = h[4 * c + 2 * e];
          float& h1 = h[4 * c + 2 * e + 1];
          h0 = fmaf(O::lo(kr[c][e]), kd, h0);
          h1 = fmaf(O::hi(kr[c][e]), kd, h1);
          hq = fmaf(h0, O::lo(qr[c][e]), fmaf(h1, O::hi(qr[c][e]), hq));
        }
      hq = reduce(hq);
      if (g8 == 0)
        static_cast<uint16_t*>(a.out)[tok * a.stride_o + static_cast<int64_t>(hv) * a.V + row] = O::narrow(hq * qs);
    }
  }
}

// One workgroup: V rows [tile ROWS, (tile + 1) ROWS) of one (request, value head); WMAX >= width staged nodes; S
// parked states per wave.
template <int K, int WMAX, int S, typename T>
__global__ __launch_bounds__(NT) void gdn_replay_kernel(const eagle4_records_args a, int tiles, int per_xcd,
                                                         int total) {
  constexpr int KB = K / 32;    // MFMA blocks over K
  constexpr int KQ = K / 4;     // K elements per lane group
  constexpr int CHK = K / 8;    // 16-byte chunks per q / k row
  constexpr int PITCH = K + 8;  // LDS row pitch in elements: consecutive rows start 4 banks apart
  constexpr int QK_IT = (WMAX * CHK + NT - 1) / NT;
  constexpr int V_IT = (WMAX * ROWS + NT - 1) / NT;
  constexpr int PE_IT = 2;  // path-table entries per thread loaded with the rest of the prologue (more: a loop)
  using O = Ops<T>;
  __shared__ __align__(16) uint16_t s_k[WMAX][PITCH];
  __shared__ __align__(16) uint16_t s_q[WMAX][PITCH];
  __shared__ uint16_t s_v[WMAX][ROWS];
  __shared__ __align__(16) float s_kh[WMAX][K];  // per node: the normalised key k ks
  __shared__ float s_dv[WMAX][ROWS];   // per node and row: delta (the record's), read again by the node's children
  __shared__ float s_oq[WMAX][ROWS];   // per node and row: decay qs (h~_parent q), the output less its delta term
  __shared__ float4 s_nd[WMAX];  // per node: decay ks, beta, decay qs, ks qs (k . q)
  __shared__ float2 s_gk[WMAX];  // per node: decay, ks
  __shared__ float2 s_g[WMAX];   // per node: decay, beta
  __shared__ int s_par[64];
  __shared__ __align__(4) uint8_t s_ch[WMAX + 1][WMAX];  // row p + 1: the children of node p in order (0xff: none)

  // Work item: consecutive items share a request and key head; the hardware deals workgroups to the 8 XCDs in turn,
  // so item = (block % 8) * per_xcd + block / 8 gives each XCD a contiguous run.
  const int w = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
  if (w >= total) return;
  const int tile = w % tiles, pair = w / tiles;
  const int hv = pair % a.HV, n = pair / a.HV;
  const int ih = hv / (a.HV / a.H);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r16 = lane & 15, g = lane >> 4;
  const int row0 = tile * ROWS;
  const int wrow = wave * 16 + r16;            // the lane's row within the workgroup
  const bool wave_on = row0 + wave * 16 < a.V;  // V % 16 == 0: a wave's rows are all inside or all past V

  const int64_t bos = uni64(e4::ld(a.query_start_loc, n));
  const int T_ = static_cast<int>(uni64(e4::ld(a.query_start_loc, n + 1)) - bos);
  const int rec_row = static_cast<int>(uni64(e4::ld(a.record_indices, n)));
  const int idx = static_cast<int>(uni64(e4::ld(a.state_indices, n)));
  const uint32_t A_raw = load_raw(a.A_log, hv, a.A_log_dtype);
  const uint32_t dt_raw = load_raw(a.dt_bias, hv, a.dt_bias_dtype);
  if (T_ <= 0) return;
  const float A = -expf(widen_raw(A_raw, a.A_log_dtype));
  const float dt_bias = widen_raw(dt_raw, a.dt_bias_dtype);
  if (rec_row < 0) {  // a request without records never reloads a parent: one chain, no rounding
    if (wave_on) chain_walk<K, T>(a, bos, T_, idx, hv, ih, row0 + wave * 16, lane, A, dt_bias);
    return;
  }
  const int Tn = T_ < a.width ? T_ : a.width;  // a tree has at most width (<= WMAX) rows

  // ---- prologue: every load in flight before the first wait --------------------------------------------------------
  // the wave's 16 rows of the pool state in the operand layout, through a buffer resource that is empty for a negative
  // slot index (zeros: the zero initial state, :73-75) or a wave past V
  const char* h0_base = static_cast<const char*>(a.state) +
                        ((idx >= 0 ? static_cast<int64_t>(idx) * a.stride_state : 0) +
                         (static_cast<int64_t>(hv) * a.V + row0 + wave * 16) * K) * 2;
  const __amdgpu_buffer_rsrc_t h0_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<char*>(h0_base), 0, idx >= 0 && wave_on ? 16 * K * 2 : 0, 0x00020000);
  auto load_h0 = [&](u32x4 (&Hc)[KB]) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      Hc[kb] = __builtin_bit_cast(u32x4,
                                  __builtin_amdgcn_raw_buffer_load_b128(h0_rs, (r16 * K + g * KQ + 8 * kb) * 2, 0, 0));
  };
  u32x4 H[KB];
  load_h0(H);
  u32x4 kr[QK_IT], qr[QK_IT];
  uint16_t vr[V_IT];
#pragma unroll
  for (int it = 0; it < QK_IT; ++it) {  // every load issued (past the tree: its last node again), stored if inside
    const int i = tid + it * NT;
    const int t = i / CHK < Tn ? i / CHK : Tn - 1, ch = i % CHK;
    const int64_t tok = bos + t;
    kr[it] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.k) + tok * a.stride_k +
                                              static_cast<int64_t>(ih) * K + 8 * ch);
    qr[it] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.q) + tok * a.stride_q +
                                              static_cast<int64_t>(ih) * K + 8 * ch);
  }
#pragma unroll
  for (int it = 0; it < V_IT; ++it) {
    const int i = tid + it * NT;
    const int t = i / ROWS < Tn ? i / ROWS : Tn - 1, r = i % ROWS;
    const int vrow = row0 + r < a.V ? row0 + r : a.V - 1;
    vr[it] = static_cast<const uint16_t*>(a.v)[(bos + t) * a.stride_v + static_cast<int64_t>(hv) * a.V + vrow];
  }
  uint32_t ga = 0, gb = 0;
  if (tid < Tn) {
    ga = load_raw(a.a, (bos + tid) * a.stride_a + hv, a.gate_dtype);
    gb = load_raw(a.b, (bos + tid) * a.stride_b + hv, a.gate_dtype);
  }
  // The tree from the path table: every entry (d > 0) of a path names the entry before it as its parent (:77-80);
  // nodes on no path are never visited (the replay writes nothing for them).
  const int D = a.width, PD = a.num_paths * a.width;
  const int32_t* paths = static_cast<const int32_t*>(a.tree_paths.ptr) + n * a.tree_paths.s0;
  int pL[PE_IT], ptok[PE_IT], pprev[PE_IT], pd[PE_IT];
  auto path_entry = [&](int i, int& L, int& tok, int& prev, int& d) {
    L = 0;
    tok = -1;
    prev = -1;
    d = 0;
    if (i < PD) {
      const int p = i / D;
      d = i % D;
      const int32_t* prow = paths + p * a.tree_paths.s1;
      L = prow[0];
      tok = prow[2 + d];
      if (d > 0) prev = prow[1 + d];
    }
  };
#pragma unroll
  for (int j = 0; j < PE_IT; ++j) path_entry(tid + j * NT, pL[j], ptok[j], pprev[j], pd[j]);
  if (tid < 64) s_par[tid] = -2;
  for (int i = tid; i < (WMAX + 1) * WMAX / 4; i += NT) reinterpret_cast<uint32_t*>(&s_ch[0][0])[i] = ~0u;
  __syncthreads();

  // ---- staging ------------------------------------------------------------------------------------------------------
  auto set_parent = [&](int L, int tok, int prev, int d) {
    if (d < L && tok >= 0 && tok < Tn && prev >= -1 && prev < Tn && prev != tok) s_par[tok] = prev;
  };
#pragma unroll
  for (int j = 0; j < PE_IT; ++j) set_parent(pL[j], ptok[j], pprev[j], pd[j]);
  for (int base = PE_IT * NT; base < PD; base += NT) {
    int L, tok, prev, d;
    path_entry(base + tid, L, tok, prev, d);
    set_parent(L, tok, prev, d);
  }
#pragma unroll
  for (int it = 0; it < QK_IT; ++it) {
    const int i = tid + it * NT;
    if (i < Tn * CHK) {
      const int t = i / CHK, ch = i % CHK;
      *reinterpret_cast<u32x4*>(&s_k[t][8 * ch]) = kr[it];
      *reinterpret_cast<u32x4*>(&s_q[t][8 * ch]) = qr[it];
    }
  }
#pragma unroll
  for (int it = 0; it < V_IT; ++it) {
    const int i = tid + it * NT;
    if (i < Tn * ROWS) s_v[i / ROWS][i % ROWS] = vr[it];
  }
  if (tid < Tn) s_g[tid] = gate_of(ga, gb, a.gate_dtype, 1.0f, 20.0f, A, dt_bias);  // decay, beta (:115-140)
  __syncthreads();

  // The tree in every wave: lane i holds node i's parent (-1 a root, -2 not in the tree) and its children. Wave 0 also
  // lists every node's children in order (s_ch), so a lane finds the children it serves with one LDS read.
  const int par = lane < Tn ? s_par[lane] : -2;
  uint64_t kids = 0;
  for (int i = 0; i < Tn; ++i) {
    const uint64_t m = __ballot(par == i);
    if (lane == i) kids = m;
  }
  const uint64_t roots = __ballot(par == -1);
  const uint64_t internal = __ballot(kids != 0);
  {
    const int src = par >= 0 ? par : lane;  // every lane takes part in the shuffles
    const uint32_t lo = static_cast<uint32_t>(__shfl(static_cast<int>(kids & 0xffffffffu), src));
    const uint32_t hi = static_cast<uint32_t>(__shfl(static_cast<int>(kids >> 32), src));
    const uint64_t sib = par == -1 ? roots : (static_cast<uint64_t>(hi) << 32) | lo;
    if (wave == 0 && par >= -1)
      s_ch[par + 1][__builtin_popcountll(sib & ((1ull << lane) - 1))] = static_cast<uint8_t>(lane);
  }

  // per node: |q|^2, |k|^2 and k . q over K (:147-150), LPN0 adjacent threads a node, the first LPN of them each
  // summing a contiguous run
  {
    constexpr int LPN0 = NT / WMAX;
    constexpr int LPN = LPN0 < K / 4 ? LPN0 : K / 4;
    constexpr int PER = K / LPN;
    static_assert(PER % 4 == 0 && LPN0 <= 16, "norm split");
    const int t = tid / LPN0, part = tid % LPN0;
    float qq = 0.f, kk = 0.f, kq = 0.f;
    if (t < Tn && part < LPN) {
#pragma unroll
      for (int c = 0; c < PER / 4; ++c) {
        const uint2 xk = *reinterpret_cast<const uint2*>(&s_k[t][part * PER + 4 * c]);
        const uint2 xq = *reinterpret_cast<const uint2*>(&s_q[t][part * PER + 4 * c]);
        const uint32_t wk[2] = {xk.x, xk.y}, wq[2] = {xq.x, xq.y};
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float k0 = O::lo(wk[e]), k1 = O::hi(wk[e]);
          const float q0 = O::lo(wq[e]), q1 = O::hi(wq[e]);
          kk = fmaf(k0, k0, fmaf(k1, k1, kk));
          qq = fmaf(q0, q0, fmaf(q1, q1, qq));
          kq = fmaf(k0, q0, fmaf(k1, q1, kq));
        }
      }
    }
    kk = e4::group_sum<LPN0>(kk);
    qq = e4::group_sum<LPN0>(qq);
    kq = e4::group_sum<LPN0>(kq);
    const float ks = 1.0f / sqrtf(kk + 1e-6f);
    if (t < Tn && part < LPN) {  // the normalised key, fp32 (what the record keeps and the state update adds)
#pragma unroll
      for (int c = 0; c < PER / 4; ++c) {
        const uint2 xk = *reinterpret_cast<const uint2*>(&s_k[t][part * PER + 4 * c]);
        *reinterpret_cast<float4*>(&s_kh[t][part * PER + 4 * c]) =
            make_float4(O::lo(xk.x) * ks, O::hi(xk.x) * ks, O::lo(xk.y) * ks, O::hi(xk.y) * ks);
      }
    }
    if (t < Tn && part == 0) {
      const float2 gt = s_g[t];
      const float qs = a.scale / sqrtf(qq + 1e-6f);
      s_nd[t] = make_float4(gt.x * ks, gt.y, gt.x * qs, ks * qs * kq);
      s_gk[t] = make_float2(gt.x, ks);
    }
  }
  __syncthreads();

  float* const rec = a.records + static_cast<int64_t>(rec_row) * a.stride_records_row;
  // the records' normalised keys and decays, once per (node, value head): the first tile's workgroup
  if (tile == 0) {
    for (int i = tid; i < Tn * (K / 4); i += NT) {
      const int t = i / (K / 4), k4 = 4 * (i % (K / 4));
      if (s_par[t] != -2) {
        float* p = rec + (static_cast<int64_t>(t) * a.HV + hv) * a.rec + a.V + k4;
        *reinterpret_cast<float4*>(p) = *reinterpret_cast<const float4*>(&s_kh[t][k4]);
        if (k4 == 0) p[K] = s_gk[t].x;
      }
    }
  }
  // ---- the tree walk (waves inside V): deltas and output terms gather in LDS, stored at the end --------------------
  // The children of node u (-1: the roots) from its rounded state Hc, eight per pass: one MFMA pass gives h~ k_j
  // (operand rows 0-7) and h~ q_j (rows 8-15); lane (g, r16) receives element r of row 4 g + r for V row r16, i.e.
  // h~ k (g < 2) or h~ q (g >= 2) of child 4 (g % 2) + r of the pass.
  auto serve = [&](int u, int nch, const u32x4 (&Hc)[KB]) {
    for (int base = 0; base < nch; base += 8) {
      const uint8_t* list = &s_ch[u + 1][base];
      const int mine = list[r16 & 7];  // the child whose k (r16 < 8) or q this lane's operand row holds
      const uint32_t cw = *reinterpret_cast<const uint32_t*>(list + 4 * (g & 1));  // the lane's 4 result children
      int c[4];
      float4 nd[4];
      float vv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int x = (cw >> (8 * r)) & 0xff;
        c[r] = x == 0xff ? -1 : x;
        const int cc = x == 0xff ? 0 : x;
        nd[r] = s_nd[cc];
        vv[r] = O::lo(s_v[cc][wrow]);
      }
      const uint16_t* src = (r16 < 8 ? &s_k[0][0] : &s_q[0][0]) + (mine == 0xff ? 0 : mine) * PITCH + g * KQ;
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        u32x4 x = *reinterpret_cast<const u32x4*>(src + 8 * kb);
        if (mine == 0xff) x = u32x4{0u, 0u, 0u, 0u};
        acc = O::mma(x, Hc[kb], acc);
      }
      // lanes g < 2: delta = (v - decay ks h~ k) beta; lanes g >= 2: decay qs h~ q (the output less delta ks qs k.q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = g < 2 ? (vv[r] - nd[r].x * acc[r]) * nd[r].y : nd[r].z * acc[r];
        if (c[r] >= 0) (g < 2 ? s_dv : s_oq)[c[r]][wrow] = x;
      }
    }
    lds_order();
  };
  // Hc <- round(decay_j Hc + k^_j delta_j^T): node j's rounded state from its parent's
  auto advance = [&](u32x4 (&Hc)[KB], int j) {
    const float decay = s_gk[j].x;
    const float dv = s_dv[j][wrow];
    const float* kp = &s_kh[j][g * KQ];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const float4 k0 = *reinterpret_cast<const float4*>(kp + 8 * kb);
      const float4 k1 = *reinterpret_cast<const float4*>(kp + 8 * kb + 4);
      const float kh[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      uint32_t nw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t hw = Hc[kb][e];
        nw[e] = O::pack(fmaf(kh[2 * e], dv, O::lo(hw) * decay), fmaf(kh[2 * e + 1], dv, O::hi(hw) * decay));
      }
      Hc[kb] = u32x4{nw[0], nw[1], nw[2], nw[3]};
    }
  };

  u32x4 st[S][KB];
  int sid[S];
#pragma unroll
  for (int s = 0; s < S; ++s) sid[s] = -3;
  int sp = 0;
  auto push = [&](int u) {
#pragma unroll
    for (int s = S - 1; s > 0; --s) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) st[s][kb] = st[s - 1][kb];
      sid[s] = sid[s - 1];
    }
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) st[0][kb] = H[kb];
    sid[0] = u;
    sp = sp < S ? sp + 1 : S;
  };
  auto top_id = [&]() { return sp > 0 ? sid[0] : -3; };
  auto pop = [&]() {
#pragma unroll
    for (int s = 0; s + 1 < S; ++s) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) st[s][kb] = st[s + 1][kb];
      sid[s] = sid[s + 1];
    }
    sid[S - 1] = -3;
    --sp;
  };
  // H <- the rounded state of node p (-1: the pool state): the stack's top, or its root path replayed
  auto restore = [&](int p) {
    if (p >= 0 && top_id() == p) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) H[kb] = st[0][kb];
      return;
    }
    load_h0(H);  // the pool state again (rare: a later root, or a parked state dropped from the stack)
    settle_loads();
    if (p < 0) return;
    int pv = -1, len = 0;  // lane d: the d-th ancestor-or-self of p
    for (int x = p; x >= 0 && len < 64; x = readlane(par, x)) {
      if (lane == len) pv = x;
      ++len;
    }
    for (int d = len - 1; d >= 0; --d) advance(H, readlane(pv, d));
  };

  // Depth first over the internal nodes: serve a node's children, then step into its first child that has children
  // of its own, or climb to the nearest ancestor with such a child left and take up that ancestor's state.
  int u = -1;
  for (int it = 0; wave_on && it <= Tn; ++it) {
    const uint64_t C = u < 0 ? roots : readlane64(kids, u);
    serve(u, __builtin_popcountll(C), H);
    const uint64_t ik = C & internal;
    int j = -1;
    if (ik != 0) {
      j = static_cast<int>(__builtin_ctzll(ik));
      if (u >= 0 && (ik & (ik - 1)) != 0) push(u);  // more such children later: park the state
    } else {
      for (int x = u, hops = 0; x >= 0 && hops < 64; ++hops) {
        const int p = readlane(par, x);
        const uint64_t above = x == 63 ? 0ull : ~0ull << (x + 1);
        const uint64_t sib = (p < 0 ? roots : readlane64(kids, p)) & internal & above;
        if (sib != 0) {
          j = static_cast<int>(__builtin_ctzll(sib));
          restore(p);
          if ((sib & (sib - 1)) == 0 && p >= 0 && top_id() == p) pop();  // its last one: unpark
          break;
        }
        x = p;
      }
    }
    if (j < 0) break;
    advance(H, j);
    u = j;
  }
  __syncthreads();

  // ---- every tree node's record delta and output, 4 rows a thread (:95-101) ----------------------------------------
  uint16_t* const out = static_cast<uint16_t*>(a.out) + bos * a.stride_o + static_cast<int64_t>(hv) * a.V + row0;
  for (int i = tid; i < Tn * (ROWS / 4); i += NT) {
    const int t = i / (ROWS / 4), r = 4 * (i % (ROWS / 4));
    if (s_par[t] == -2 || row0 + r >= a.V) continue;
    const float4 dv = *reinterpret_cast<const float4*>(&s_dv[t][r]);
    const float4 oq = *reinterpret_cast<const float4*>(&s_oq[t][r]);
    const float w = s_nd[t].w;
    *reinterpret_cast<float4*>(rec + (static_cast<int64_t>(t) * a.HV + hv) * a.rec + row0 + r) = dv;
    const u32x2 o = {O::pack(fmaf(dv.x, w, oq.x), fmaf(dv.y, w, oq.y)),
                     O::pack(fmaf(dv.z, w, oq.z), fmaf(dv.w, w, oq.w))};
    *reinterpret_cast<u32x2*>(out + t * a.stride_o + r) = o;
  }
}

template <int K, int WMAX, int S>
int launch_k(const eagle4_records_args& a, hipStream_t s) {
  const int tiles = e4::ceil_div(a.V, ROWS);
  const int64_t total = static_cast<int64_t>(a.N) * a.HV * tiles;
  if (total > (int64_t(1) << 30)) return EAGLE4_NOT_COVERED;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  const dim3 grid(8 * per_xcd);
  if (a.state_dtype == EAGLE4_BF16)
    gdn_replay_kernel<K, WMAX, S, e4::Bf16><<<grid, NT, 0, s>>>(a, tiles, per_xcd, static_cast<int>(total));
  else
    gdn_replay_kernel<K, WMAX, S, e4::F16><<<grid, NT, 0, s>>>(a, tiles, per_xcd, static_cast<int>(total));
  return E4_LAUNCH_STATUS();
}

template <int K, int S>
int launch_w(const eagle4_records_args& a, hipStream_t s) {
  if (a.width <= 16) return launch_k<K, 16, S>(a, s);
  if constexpr (K == 256)  // the staged rows of 64 nodes would not fit LDS: up to 32
    return a.width <= 32 ? launch_k<K, 32, S>(a, s) : EAGLE4_NOT_COVERED;
  else
    return launch_k<K, 64, S>(a, s);
}

}  // namespace

namespace e4replay {

// The path replay on the matrix cores when it covers the call: a path table, 16-bit q / k / v, output and pool of one
// dtype (the MFMA operands exact), a key dim of 32 .. 256 (a multiple of 32), a value dim that is a multiple of 16,
// trees of <= 64 nodes (<= 32 at K = 256), 16-byte aligned q / k rows, pool slots and records, 8-byte aligned output rows. Returns
// EAGLE4_NOT_COVERED (nothing launched) otherwise.
int launch(const eagle4_records_args& a, hipStream_t s) {
  const auto al = [](const void* p, int64_t bytes) { return reinterpret_cast<uintptr_t>(p) % bytes == 0; };
  if (!a.path_replay || a.in_dtype != a.state_dtype || a.out_dtype != a.in_dtype ||
      (a.in_dtype != EAGLE4_BF16 && a.in_dtype != EAGLE4_F16) ||
      a.width < 1 || a.width > 64 || a.V % 16 || a.V < 16 || a.HV % a.H || a.rec < a.V + a.K + 1 || a.stride_q % 8 ||
      a.stride_k % 8 || a.stride_state % 8 || !al(a.q, 16) || !al(a.k, 16) || !al(a.state, 16) || a.rec % 4 ||
      a.stride_records_row % 4 || !al(a.records, 16) || a.stride_o % 4 || !al(a.out, 8) ||
      a.tree_paths.dtype != EAGLE4_I32)
    return EAGLE4_NOT_COVERED;
  switch (a.K) {
    case 32: return launch_w<32, 4>(a, s);
    case 64: return launch_w<64, 4>(a, s);
    case 128: return launch_w<128, 2>(a, s);
    case 256: return launch_w<256, 2>(a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}

}  // namespace e4replay
