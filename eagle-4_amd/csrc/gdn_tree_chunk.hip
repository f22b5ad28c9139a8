// GDN tree chunk form on the gfx950 matrix cores (kernels/gdn_tree_records.py:276-361, 496-579): the records
// contract's verify without per-node rounding, for trees of at most 16 nodes, solved in closed form per (request,
// value head) instead of walked node by node:
//
//   R = strict-ancestor closure of the parent links,   G_t = product of exp(g) along t's root path,
//   L = diag(beta) (R o G_t/G_j o K K^T),               D = (I + L)^-1 diag(beta) (V - diag(G) K S0^T),
//   O = diag(G) Q S0^T + ((R + I) o G_t/G_j o Q K^T) D,
//
// with Q, K the normalised queries / keys (scale folded into Q) and S0 the request's [V, K] pool state. D is the
// record's delta, so the records hold (D, K, exp(g)) and the commit replays them.
//
// One wave per (request, value head, slice of 16 NTL value columns), 16 nodes on the 16 rows of the 16x16 MFMA
// accumulator (lane (g, c), element r: row 4 g + r, column c):
//   - everything the wave reads is issued first: parents, gates, q / k rows, v, the pool slice;
//   - K K^T, K Q^T and Q Q^T on v_mfma_f32_16x16x32_bf16 from the raw bf16 rows (products exact, fp32 sums); the
//     squared norms are the diagonals, and the norms enter as per-row factors;
//   - per node (lane c): decay / beta, and by pointer jumping over the parent links the ancestor set (a 16-bit mask)
//     and the root-path log2-decay sum log2 G; the decay ratios are then hardware exp2 of log2 differences;
//   - L, L^T and W^T masked and scaled from K K^T and K Q^T;
//   - (I + L)^-1 = (I - L)(I + L^2)(I + L^4)(I + L^8) (L is strictly lower in the ancestor order, L^16 = 0) by 8
//     products on v_mfma_f32_16x16x4f32, kept transposed as the left operand of D = Tinv rhs;
//   - per 16-column tile, K S0^T and Q S0^T on the bf16 MFMA with the pool state split into exact bf16 terms
//     (1 for a bf16 pool, 2 for fp16, 3 for fp32), then rhs, D and O on the fp32 MFMA.
// Tile u of a wave covers the columns v0 + NTL c + u, so each lane ends with NTL adjacent columns of every row it
// holds: the records' deltas leave as 16 NTL-byte runs per lane.
// Work items are ordered so that the waves of one request's key head (its value heads and column slices) run on
// one XCD and share the q / k rows in its L2.

#include "gdn_walk.h"

namespace e4chunk {
int launch(const eagle4_records_args& a, hipStream_t s) __attribute__((visibility("hidden")));
}

namespace {

using namespace e4walk;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int NP = 16;  // nodes per request: the rows of one MFMA tile

E4_DEV f32x4_t mma_bf16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// X Y for 16 x 16 fp32 matrices in the accumulator layout, X passed transposed: block kb of the 16x16x4 MFMA
// contracts over k = 4 g + kb, for which a lane's A operand X[c][4 g + kb] is element kb of its X^T and its B operand
// Y[4 g + kb][c] element kb of its Y.
E4_DEV f32x4_t mm(f32x4_t xt, f32x4_t y) {
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xt[kb], y[kb], acc, 0, 0, 0);
  return acc;
}

// Loads whose width does not depend on a runtime dtype, so every dtype takes one code path and the compiler has no
// join at which to wait for loads in flight. A float input: the aligned 32-bit word holding element i (an allocation
// holds whole words) and the shift that brings the element to the low bits.
struct Word {
  uint32_t w;
  uint32_t sh;
};
E4_DEV Word word_of(const void* p, int64_t i, int dtype) {
  const int64_t byte = dtype == EAGLE4_F32 ? 4 * i : 2 * i;
  const uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const char*>(p) + (byte & ~int64_t(3)));
  return {w, static_cast<uint32_t>(byte & 2) * 8u};
}
E4_DEV float widen_word(const Word& x, int dtype) {
  const uint32_t r = dtype == EAGLE4_F32 ? x.w : (x.w >> x.sh) & 0xffffu;
  return widen_raw(r, dtype);
}
// An integer table entry through its low 32 bits: int32, or int64 holding a value in int32 range (token offsets,
// slots, rows, parents).
E4_DEV int32_t entry(const eagle4_itab& t, int64_t i, int64_t j = 0) {
  const int64_t off = (i * t.s0 + j * t.s1) * (t.dtype == EAGLE4_I64 ? 8 : 4);
  return *reinterpret_cast<const int32_t*>(static_cast<const char*>(t.ptr) + off);
}

E4_DEV float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
E4_DEV float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
// Two fp32 values whose low 16 bits are zero (exact bf16 values) packed as bf16 elements 2 i, 2 i + 1.
E4_DEV uint32_t pack2(float x0, float x1) { return (__float_as_uint(x0) >> 16) | (__float_as_uint(x1) & 0xffff0000u); }
E4_DEV float trunc_bf16(float x) { return __uint_as_float(__float_as_uint(x) & 0xffff0000u); }

// The pool state as exact bf16 terms. A lane's slice of one tile and K block is 8 consecutive state elements (one
// row, k = 32 kb + 8 g ...); term 0 keeps the leading 8 significand bits (truncated), each further term those of what
// the earlier ones left, so the terms sum to the element exactly (fp16: 11 bits, 2 terms; fp32: 24 bits, 3 terms).
template <typename Tpool>
struct PoolTerms {
  static constexpr bool kF32 = sizeof(typename Tpool::storage) == 4;
  static constexpr int N = kF32 ? 3 : (Tpool::code == EAGLE4_F16 ? 2 : 1);
  static constexpr int WORDS = kF32 ? 2 : 1;  // uint4 per lane per (tile, K block)
  static E4_DEV void split(const uint4 (&raw)[WORDS], uint4 (&t)[N]) {
    if constexpr (N == 1) {
      t[0] = raw[0];
    } else {
      float x[8];
      if constexpr (kF32) {
        const uint32_t w[8] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w, raw[1].x, raw[1].y, raw[1].z, raw[1].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = __uint_as_float(w[e]);
      } else {
        const uint32_t w[4] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[2 * e] = e4::f16_to_f32(static_cast<uint16_t>(w[e] & 0xffffu));
          x[2 * e + 1] = e4::f16_to_f32(static_cast<uint16_t>(w[e] >> 16));
        }
      }
      uint32_t p[N][4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float r0 = x[2 * e], r1 = x[2 * e + 1];
#pragma unroll
        for (int s = 0; s < N; ++s) {
          const float t0 = trunc_bf16(r0), t1 = trunc_bf16(r1);
          p[s][e] = pack2(t0, t1);
          r0 -= t0;  // exact: the bits below the kept ones
          r1 -= t1;
        }
      }
#pragma unroll
      for (int s = 0; s < N; ++s) t[s] = make_uint4(p[s][0], p[s][1], p[s][2], p[s][3]);
    }
  }
};

// NTL adjacent 16-bit elements (v inputs) as raw words.
template <int NTL>
struct Run16 {
  uint32_t w[(NTL + 1) / 2];
  E4_DEV void load(const uint16_t* p) {
    if constexpr (NTL == 4) {
      const uint2 x = *reinterpret_cast<const uint2*>(p);
      w[0] = x.x;
      w[1] = x.y;
    } else if constexpr (NTL == 2) {
      w[0] = *reinterpret_cast<const uint32_t*>(p);
    } else {
      w[0] = *p;
    }
  }
  E4_DEV float at(int u) const { return (u & 1) ? hi_bf16(w[u >> 1]) : lo_bf16(w[u >> 1]); }
};

template <int NTL>
E4_DEV void store_run_f32(float* p, const float (&x)[NTL]) {
  if constexpr (NTL == 4)
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  else if constexpr (NTL == 2)
    *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
  else
    *p = x[0];
}

template <int NTL>
E4_DEV void store_run_out(void* base, int64_t i, int dtype, const float (&x)[NTL]) {
  if (dtype == EAGLE4_F32) {
    store_run_f32<NTL>(static_cast<float*>(base) + i, x);
    return;
  }
  uint16_t h[NTL];
#pragma unroll
  for (int u = 0; u < NTL; ++u) h[u] = dtype == EAGLE4_BF16 ? e4::f32_to_bf16(x[u]) : e4::f32_to_f16(x[u]);
  uint16_t* p = static_cast<uint16_t*>(base) + i;
  if constexpr (NTL == 4)
    *reinterpret_cast<uint2*>(p) = make_uint2(h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16));
  else if constexpr (NTL == 2)
    *reinterpret_cast<uint32_t*>(p) = h[0] | (uint32_t(h[1]) << 16);
  else
    *p = h[0];
}

template <int K, int NTL, typename Tpool>
__global__ __launch_bounds__(64) void gdn_chunk_kernel(const eagle4_records_args a, int slices, int per_xcd,
                                                        int total) {
  constexpr int KB = K / 32;
  using PT = PoolTerms<Tpool>;
  __shared__ float4 s_nd[NP];    // per node: ks, qs, beta, log G
  __shared__ uint32_t s_anc[NP];  // per node: strict ancestors

  // Work item: consecutive items share a key head (value heads of one group, then column slices); the hardware deals
  // workgroups to the 8 XCDs in turn, so item = (block % 8) * per_xcd + block / 8 gives each XCD one contiguous run.
  const int w = static_cast<int>(blockIdx.x % 8) * per_xcd + static_cast<int>(blockIdx.x / 8);
  if (w >= total) return;
  const int slice = w % slices, pair = w / slices;
  const int hv = pair % a.HV, n = pair / a.HV;
  const int ih = hv / (a.HV / a.H);
  const int lane = threadIdx.x, c = lane & 15, g = lane >> 4;

  // the request's table entries and the head's gate constants, all in flight together
  const int qs0 = entry(a.query_start_loc, n), qs1 = entry(a.query_start_loc, n + 1);
  const int rec_row = uni(entry(a.record_indices, n));
  const int idx = uni(entry(a.state_indices, n));
  const Word A_w = word_of(a.A_log, hv, a.A_log_dtype);
  const Word dt_w = word_of(a.dt_bias, hv, a.dt_bias_dtype);
  const int64_t bos = uni(qs0);
  int T = uni(qs1) - uni(qs0);
  T = T < a.width ? T : a.width;  // a tree has at most width (<= 16) rows
  if (T <= 0) return;

  // ---- every other load before the first wait -------------------------------------------------------------------
  const int ct = c < T ? c : T - 1;  // lanes past the tree read its last node (finite values, masked below)
  const int64_t tok = bos + ct;
  const int par_raw = entry(a.parent, n, ct);
  const Word ga = word_of(a.a, tok * a.stride_a + hv, a.gate_dtype);
  const Word gb = word_of(a.b, tok * a.stride_b + hv, a.gate_dtype);
  uint4 qr[KB], kr[KB];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + tok * a.stride_q + ih * K + 8 * g;
    const uint16_t* kp = static_cast<const uint16_t*>(a.k) + tok * a.stride_k + ih * K + 8 * g;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      qr[kb] = *reinterpret_cast<const uint4*>(qp + 32 * kb);
      kr[kb] = *reinterpret_cast<const uint4*>(kp + 32 * kb);
    }
  }
  // v before the pool slice: loads complete in order, and the first tile needs v but only its own slice part
  const int v0 = slice * 16 * NTL;
  Run16<NTL> vr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * g + r;
    const int64_t ti = bos + (i < T ? i : T - 1);
    vr[r].load(static_cast<const uint16_t*>(a.v) + ti * a.stride_v + static_cast<int64_t>(hv) * a.V + v0 + NTL * c);
  }
  // The pool slice (rows v0 .. v0 + 16 NTL of the request's slot) through a buffer resource whose range is the slice,
  // or empty for a negative slot index: its loads then return zeros, the zero initial state (:341-345), with no
  // branch around them.
  using PS = typename Tpool::storage;
  constexpr int kSliceBytes = 16 * NTL * K * static_cast<int>(sizeof(PS));
  const char* slot = static_cast<const char*>(a.state) +
                     ((idx >= 0 ? static_cast<int64_t>(idx) * a.stride_state : 0) +
                      (static_cast<int64_t>(hv) * a.V + v0) * K) * static_cast<int64_t>(sizeof(PS));
  const __amdgpu_buffer_rsrc_t srsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(slot), 0, idx >= 0 ? kSliceBytes : 0, 0x00020000);
  uint4 sraw[NTL][KB][PT::WORDS];
#pragma unroll
  for (int u = 0; u < NTL; ++u)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int q = 0; q < PT::WORDS; ++q) {
        const int off = ((NTL * c + u) * K + 32 * kb + 8 * g) * static_cast<int>(sizeof(PS)) + 16 * q;
        sraw[u][kb][q] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(srsrc, off, 0, 0));
      }
  // keep the scheduler from sinking these loads below the per-node math that waits for the q / k rows
  __builtin_amdgcn_sched_barrier(0);

  // ---- node x node products; their diagonals are the squared norms ---------------------------------------------------
  f32x4_t KK = {0.f, 0.f, 0.f, 0.f}, KQ = {0.f, 0.f, 0.f, 0.f}, QQ = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    KK = mma_bf16(kr[kb], kr[kb], KK);  // KK[i][j] = k_i . k_j
    KQ = mma_bf16(kr[kb], qr[kb], KQ);  // KQ[i][j] = k_i . q_j
    QQ = mma_bf16(qr[kb], qr[kb], QQ);  // QQ[i][j] = q_i . q_j
  }

  // ---- per node (lane c): gates, ancestors, root-path log decay -----------------------------------------------------
  const float A = -expf(widen_word(A_w, a.A_log_dtype));
  const float dt_bias = widen_word(dt_w, a.dt_bias_dtype);
  const uint32_t ga_raw = a.gate_dtype == EAGLE4_F32 ? ga.w : (ga.w >> ga.sh) & 0xffffu;
  const uint32_t gb_raw = a.gate_dtype == EAGLE4_F32 ? gb.w : (gb.w >> gb.sh) & 0xffffu;
  const float2 gt = gate_of(ga_raw, gb_raw, a.gate_dtype, 1.0f, 20.0f, A, dt_bias);
  const float decay = c < T ? gt.x : 1.0f, beta = c < T ? gt.y : 0.0f;  // past the tree: exp(g) 1, beta 0 (:316-317)
  // a parent outside the tree (or the node itself) makes the node a root
  const int par = c > 0 && c < T && par_raw >= 0 && par_raw < T && par_raw != c ? par_raw : -1;
  // pointer jumping: after round j, anc holds the ancestors at distance 1 .. 2^j, lsum the log2 decays of the node and
  // its ancestors at distance < 2^j, jmp the ancestor at distance 2^j (-1 past the root); depth < 16 needs 4 rounds.
  // Decay ratios are then powers of two of log2 differences (the hardware exp2 / log2, ~1 ulp).
  uint32_t anc = par >= 0 ? 1u << par : 0u;
  int jmp = par;
  float lsum = __builtin_amdgcn_logf(fmaxf(decay, 1e-30f));
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int src = jmp >= 0 ? jmp : c;
    const uint32_t anc_j = static_cast<uint32_t>(__shfl(static_cast<int>(anc), src, 16));
    const int jmp_j = __shfl(jmp, src, 16);
    const float l_j = __shfl(lsum, src, 16);
    if (jmp >= 0) {
      anc |= anc_j;
      lsum += l_j;
      jmp = jmp_j;
    }
  }
  const float logG = lsum;  // log2 G
  // node c's squared norms sit on the diagonals at lane (c / 4, c), element c % 4; that lane publishes the node
  const int rc = c & 3;
  const float kk = rc == 0 ? KK[0] : rc == 1 ? KK[1] : rc == 2 ? KK[2] : KK[3];
  const float qq = rc == 0 ? QQ[0] : rc == 1 ? QQ[1] : rc == 2 ? QQ[2] : QQ[3];
  if (g == (c >> 2)) {
    s_nd[c] = make_float4(1.0f / sqrtf(kk + 1e-6f), a.scale / sqrtf(qq + 1e-6f), beta, logG);  // (:147-150)
    s_anc[c] = anc;
  }
  __syncthreads();
  const float ks = s_nd[c].x, qs = s_nd[c].y;
  // the record's key and decay (once per node and value head) leave now, ahead of the matrix work
  float* rec = a.records + static_cast<int64_t>(rec_row) * a.stride_records_row;
  if (slice == 0 && rec_row >= 0 && c < T) {
    float* p = rec + (static_cast<int64_t>(c) * a.HV + hv) * a.rec + a.V;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const uint4 x = kr[kb];
      float4* d = reinterpret_cast<float4*>(p + 32 * kb + 8 * g);
      d[0] = make_float4(lo_bf16(x.x) * ks, hi_bf16(x.x) * ks, lo_bf16(x.y) * ks, hi_bf16(x.y) * ks);
      d[1] = make_float4(lo_bf16(x.z) * ks, hi_bf16(x.z) * ks, lo_bf16(x.w) * ks, hi_bf16(x.w) * ks);
    }
    if (g == 0) p[K] = decay;
  }

  // ---- L, L^T, W^T -------------------------------------------------------------------------------------------------
  float4 nd[4];
  float Gr[4];
  f32x4_t L, LT, WT, I;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * g + r;
    nd[r] = s_nd[i];
    const uint32_t anc_i = s_anc[i];
    Gr[r] = __builtin_amdgcn_exp2f(nd[r].w);
    const bool c_above_i = (anc_i >> c) & 1u;  // c a strict ancestor of i
    const bool i_above_c = (anc >> i) & 1u;    // i a strict ancestor of c
    const float kk_n = nd[r].x * ks * KK[r];
    // L[i][c] = beta_i G_i / G_c k^_i . k^_c on strict ancestors c of i
    L[r] = c_above_i ? nd[r].z * __builtin_amdgcn_exp2f(nd[r].w - logG) * kk_n : 0.f;
    // L^T[i][c] = L[c][i];  W^T[i][c] = W[c][i] = G_c / G_i q^_c . k^_i on ancestors-or-self i of c
    const float ratio = i_above_c || i == c ? __builtin_amdgcn_exp2f(logG - nd[r].w) : 0.f;
    LT[r] = i_above_c ? beta * ratio * kk_n : 0.f;
    WT[r] = ratio * (qs * nd[r].x * KQ[r]);
    I[r] = i == c ? 1.f : 0.f;
  }
  // Tinv^T = (I + P8^T)(I + P4^T)(I + P2^T)(I - L^T), P2 = L L, P4 = P2 P2, P8 = P4 P4 (powers of L commute)
  const f32x4_t P2 = mm(LT, L), P2T = mm(L, LT);
  const f32x4_t P4 = mm(P2T, P2), P4T = mm(P2, P2T);
  const f32x4_t P8 = mm(P4T, P4);
  f32x4_t TinvT = mm(I + P2, I - LT);
  TinvT = mm(I + P4, TinvT);
  TinvT = mm(I + P8, TinvT);

  // ---- per 16-column tile: K S0^T, Q S0^T, rhs, D = Tinv rhs, O = G Q S0^T + W D ------------------------------------
  float D[4][NTL], O[4][NTL];
#pragma unroll
  for (int u = 0; u < NTL; ++u) {
    f32x4_t KS = {0.f, 0.f, 0.f, 0.f}, QS = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      uint4 st[PT::N];
      PT::split(sraw[u][kb], st);
#pragma unroll
      for (int s = 0; s < PT::N; ++s) {
        KS = mma_bf16(kr[kb], st[s], KS);
        QS = mma_bf16(qr[kb], st[s], QS);
      }
    }
    f32x4_t rhs;
#pragma unroll
    for (int r = 0; r < 4; ++r)
      rhs[r] = 4 * g + r < T ? nd[r].z * (vr[r].at(u) - Gr[r] * (nd[r].x * KS[r])) : 0.f;
    const f32x4_t Dt = mm(TinvT, rhs);
    const f32x4_t Wd = mm(WT, Dt);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      D[r][u] = Dt[r];
      O[r][u] = Gr[r] * (nd[r].y * QS[r]) + Wd[r];
    }
  }

  // ---- stores --------------------------------------------------------------------------------------------------------
  const int64_t col = static_cast<int64_t>(hv) * a.V + v0 + NTL * c;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int i = 4 * g + r;
    if (i < T) {
      store_run_out<NTL>(a.out, (bos + i) * a.stride_o + col, a.out_dtype, O[r]);
      if (rec_row >= 0) store_run_f32<NTL>(rec + (static_cast<int64_t>(i) * a.HV + hv) * a.rec + v0 + NTL * c, D[r]);
    }
  }
}

template <int K, int NTL>
int launch_pool(const eagle4_records_args& a, hipStream_t s) {
  const int slices = a.V / (16 * NTL);
  const int64_t total = static_cast<int64_t>(a.N) * a.HV * slices;
  if (total > (int64_t(1) << 30)) return EAGLE4_NOT_COVERED;
  const int per_xcd = static_cast<int>((total + 7) / 8);
  const dim3 grid(8 * per_xcd);
  const int t = static_cast<int>(total);
  if (a.state_dtype == EAGLE4_BF16)
    gdn_chunk_kernel<K, NTL, e4::Bf16><<<grid, 64, 0, s>>>(a, slices, per_xcd, t);
  else if (a.state_dtype == EAGLE4_F16)
    gdn_chunk_kernel<K, NTL, e4::F16><<<grid, 64, 0, s>>>(a, slices, per_xcd, t);
  else if constexpr (NTL < 4)  // four tiles of an fp32 slice would not fit the registers
    if (a.state_dtype == EAGLE4_F32)
      gdn_chunk_kernel<K, NTL, e4::F32><<<grid, 64, 0, s>>>(a, slices, per_xcd, t);
    else
      return EAGLE4_NOT_COVERED;
  else
    return EAGLE4_NOT_COVERED;
  return E4_LAUNCH_STATUS();
}

template <int K>
int launch_k(const eagle4_records_args& a, hipStream_t s) {
  // columns per wave: more columns per wave once there are enough waves to keep HBM busy (measured at 16 / 48 heads,
  // K = V = 128: 1 tile per wave at 1 request, 2 at 4, 4 at 16 and 32)
  const int64_t pairs = static_cast<int64_t>(a.N) * a.HV;
  const bool fp32_pool = a.state_dtype == EAGLE4_F32;
  if constexpr (K <= 128)
    if (!fp32_pool && a.V % 64 == 0 && pairs * (a.V / 64) >= 1024) return launch_pool<K, 4>(a, s);
  if (a.V % 32 == 0 && pairs * (a.V / 32) >= 512) return launch_pool<K, 2>(a, s);
  return launch_pool<K, 1>(a, s);
}

}  // namespace

namespace e4chunk {

// The chunk form on the matrix cores when it covers the call: no path table, trees of <= 16 nodes, bf16 inputs, a
// key dim that is a multiple of 32 (<= 256), value dim a multiple of 16, 16-byte aligned rows. Returns
// EAGLE4_NOT_COVERED (nothing launched) otherwise.
int launch(const eagle4_records_args& a, hipStream_t s) {
  const auto al = [](const void* p, int64_t bytes) { return reinterpret_cast<uintptr_t>(p) % bytes == 0; };
  if (a.path_replay || a.width > NP || a.in_dtype != EAGLE4_BF16 || a.V % 16 || a.stride_q % 8 || a.stride_k % 8 ||
      a.stride_v % 4 || a.stride_o % 4 || a.rec % 4 || a.stride_records_row % 4 || !al(a.q, 16) || !al(a.k, 16) ||
      !al(a.v, 8) || !al(a.out, 16) || !al(a.records, 16) || !al(a.state, 16) || a.stride_state % 8)
    return EAGLE4_NOT_COVERED;
  switch (a.K) {
    case 32: return launch_k<32>(a, s);
    case 64: return launch_k<64>(a, s);
    case 128: return launch_k<128>(a, s);
    case 256: return launch_k<256>(a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}

}  // namespace e4chunk
