// GDN records contract on gfx950 (kernels/gdn_tree_records.py): the tree verify writes per node a replay record
// (delta = v' [V], the normalised key [K], the decay exp(g)) instead of a [V, K] state snapshot, and the commit folds
// the accepted node's root path of records back into the pool.
//
// Verify (eagle4_gdn_tree_records_update). The reference replays every leaf's root path from the pool state, one
// program per path (path replay, :16-101, rounding each parent state to the pool dtype before its children read it),
// or, for fp32 pools, solves the tree in closed form (chunk form, :276-361). Both give every node the same fold over
// its root path; here one wave walks the tree depth first once, as the snapshot walk does (gdn_tree_recurrence.hip):
// a first child continues from the registers, a node with several children parks its state on a per-wave LDS stack
// for the later ones, and a parent that found the stack full is recomputed by replaying its root path from the pool
// state (there are no snapshots to reload). With path replay the tree is read from the path table (every entry names
// its predecessor as the parent) and parked states are rounded exactly as the replay rounds them; the chunk form
// reads `parent` and never rounds. The workload is the pool-state read (64 KB per request and value head at
// K = V = 128 fp32) and the walk's arithmetic; records are ~1 KB per node.
//
// Commit (eagle4_gdn_tree_records_commit, :160-272): per (V tile, request x value head, layer) the accepted node's
// root path is folded into the pool state, S <- S exp(g) + delta key^T node by node from the root, rounded to the
// pool dtype between nodes when asked.

#include "gdn_walk.h"

namespace e4chunk {
// gdn_tree_chunk.hip: the chunk form on the matrix cores (trees of <= 16 nodes, bf16 inputs)
int launch(const eagle4_records_args& a, hipStream_t s) __attribute__((visibility("hidden")));
}
namespace e4replay {
// gdn_tree_replay.hip: the rounded path replay on the matrix cores (16-bit inputs and pool of one dtype)
int launch(const eagle4_records_args& a, hipStream_t s) __attribute__((visibility("hidden")));
}

namespace {

using namespace e4walk;

// One workgroup: WAVES waves over consecutive V rows of one (request, value head); a wave owns RPT x (64 / C) rows.
template <int K, int C, int RPT, int WAVES, int S, typename Tin, typename Tpool>
__global__ __launch_bounds__(64 * WAVES) void gdn_records_walk_kernel(const eagle4_records_args a) {
  constexpr int E = K / C;
  constexpr int NJ = E / 4;
  constexpr int ROWS_WAVE = RPT * (64 / C);
  constexpr int ROWS = WAVES * ROWS_WAVE;
  constexpr int NT = 64 * WAVES;
  static_assert(E % 4 == 0 && C <= 64, "lane layout");
  using IS = typename Tin::storage;
  constexpr int TS = sizeof(IS) == 4 ? 8 : 16;                       // staged nodes
  constexpr bool kPoolExact = sizeof(typename Tpool::storage) == 4;  // an fp32 pool: rounding is the identity
  __shared__ float4 stack[WAVES][S][RPT * NJ][64];
  __shared__ __align__(16) IS s_q[TS][K];
  __shared__ __align__(16) IS s_k[TS][K];
  __shared__ IS s_v[TS][ROWS];
  __shared__ float4 s_sc[TS];
  __shared__ int s_par[64];

  const int n = blockIdx.z, hv = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane % C, rr = lane / C;
  const int ih = hv / (a.HV / a.H);
  const int row0 = blockIdx.x * ROWS;
  int rows[RPT], lrow[RPT];
#pragma unroll
  for (int s = 0; s < RPT; ++s) {
    lrow[s] = wave * ROWS_WAVE + s * (64 / C) + rr;
    rows[s] = row0 + lrow[s];
  }
  // the request's tables first, all in flight together
  const int64_t bos = uni64(e4::ld(a.query_start_loc, n));
  const int64_t eos = uni64(e4::ld(a.query_start_loc, n + 1));
  const int64_t rec_idx = uni64(e4::ld(a.record_indices, n));
  const int64_t idx = uni64(e4::ld(a.state_indices, n));
  const uint32_t A_raw = load_raw(a.A_log, hv, a.A_log_dtype);
  const uint32_t dt_raw = load_raw(a.dt_bias, hv, a.dt_bias_dtype);
  const int T = static_cast<int>(eos - bos);
  if (T <= 0) return;
  const bool chain = a.path_replay && rec_idx < 0;  // a request without records: one chain, no rounding (:51-53)
  const bool round = !kPoolExact && a.path_replay && rec_idx >= 0;
  const int Tn = chain ? T : (T < a.width ? T : a.width);  // nodes walked: a tree has at most width (<= 64) rows

  // The prologue issues every load before its first wait: the initial state (the request's pool slot, zeros for a
  // negative index, :73-75), the staged nodes' inputs, the parent table, then the path table.
  float h[RPT][E];
  u32x4 h0raw[RPT][NJ];
  const int64_t head_off = static_cast<int64_t>(hv) * a.V * K;
  auto issue_h0 = [&]() {
#pragma unroll
    for (int s = 0; s < RPT; ++s)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        h0raw[s][j] = u32x4{0u, 0u, 0u, 0u};  // zero bits: +0.0 in every dtype
        if (idx >= 0 && rows[s] < a.V)
          load_state_raw(a.state, idx * a.stride_state + head_off + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j,
                         a.state_dtype, h0raw[s][j]);
      }
  };
  auto widen_h0 = [&]() {
#pragma unroll
    for (int s = 0; s < RPT; ++s)
#pragma unroll
      for (int j = 0; j < NJ; ++j) widen_state_raw(h0raw[s][j], a.state_dtype, &h[s][4 * j]);
  };
  auto load_h0 = [&]() {
    issue_h0();
    settle_loads();
    widen_h0();
  };
  issue_h0();
  const int ts = Tn < TS ? Tn : TS;
  Staging<Tin, K, TS, ROWS, NT> stg;
  const NodeSrc src{a.q, a.k, a.v, a.a, a.b, a.stride_q, a.stride_k, a.stride_v, a.stride_a, a.stride_b,
                    a.gate_dtype, ih, hv, a.V};
  stg.issue(src, bos, ts, row0, tid);
  int par = -2;
  if (!chain && !a.path_replay && lane < Tn) par = lane == 0 ? -1 : static_cast<int>(e4::ld(a.parent, n, lane));

  // The tree. Path replay: every entry (d > 0) of a path names the entry before it as its parent (:77-80); nodes on
  // no path are never visited (the replay writes nothing for them). Chunk form: `parent`, node 0 the root.
  if (!chain && a.path_replay) {
    if (tid < 64) s_par[tid] = -2;
    __syncthreads();
    const int D = a.width, PD = a.num_paths * a.width;
    for (int base = 0; base < PD; base += 4 * NT) {  // 4 entries per thread in flight
      int L[4], tok[4], prev[4], dd[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = base + j * NT + tid;
        L[j] = 0;
        tok[j] = -1;
        prev[j] = -1;
        dd[j] = 0;
        if (i < PD) {
          const int p = i / D, d = i % D;
          const int32_t* prow = static_cast<const int32_t*>(a.tree_paths.ptr) + n * a.tree_paths.s0 + p * a.tree_paths.s1;
          dd[j] = d;
          L[j] = prow[0];
          tok[j] = prow[2 + d];
          if (d > 0) prev[j] = prow[1 + d];
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (dd[j] < L[j] && tok[j] >= 0 && tok[j] < Tn && prev[j] >= -1 && prev[j] < Tn && prev[j] != tok[j])
          s_par[tok[j]] = prev[j];
      }
    }
  }

  // ---- staging: q, k, v and the node scalars of nodes [0, ts) into LDS --------------------------------------------
  // the per-token values of the pre kernel (:104-156): softplus beta 1, threshold 20
  const float A = -expf(widen_raw(A_raw, a.A_log_dtype));
  const float dt_bias = widen_raw(dt_raw, a.dt_bias_dtype);
  stg.commit(s_q, s_k, s_v, s_sc, ts, tid, a.gate_dtype, 1.0f, 20.0f, A, dt_bias);
  widen_h0();
  __syncthreads();
  stage_norms<Tin, K, TS, NT>(s_q, s_k, s_sc, ts, tid, a.scale);
  __syncthreads();

  // lane i: node i's parent (-1 a root: starts from the pool state; -2 not in the tree), children and the roots
  uint64_t kids = 0, roots = 0;
  if (!chain) {
    if (lane < Tn) {
      if (a.path_replay)
        par = s_par[lane];
      else if (lane > 0 && (par < 0 || par >= Tn || par == lane))
        par = -1;  // outside the request: no ancestors
    }
    for (int i = 0; i < Tn; ++i) {
      const uint64_t m = __ballot(lane < Tn && par == i);
      if (lane == i) kids = m;
    }
    roots = __ballot(lane < Tn && par == -1);
  }
  settle_loads();  // the initial state and the tables

  auto fetch = [&](Node<E, RPT, Tin>& nd, int u) {
    if (u < TS) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        nd.q[j] = *reinterpret_cast<const Raw4<Tin>*>(&s_q[u][4 * c + 4 * C * j]);
        nd.k[j] = *reinterpret_cast<const Raw4<Tin>*>(&s_k[u][4 * c + 4 * C * j]);
      }
#pragma unroll
      for (int s = 0; s < RPT; ++s) nd.v[s] = s_v[u][lrow[s]];
      nd.sc = s_sc[u];
    } else {
      const int64_t tok = bos + u;
      const IS* q = static_cast<const IS*>(a.q) + tok * a.stride_q + static_cast<int64_t>(ih) * K;
      const IS* k = static_cast<const IS*>(a.k) + tok * a.stride_k + static_cast<int64_t>(ih) * K;
      float qq = 0.f, kk = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        nd.q[j] = *reinterpret_cast<const Raw4<Tin>*>(q + 4 * c + 4 * C * j);
        nd.k[j] = *reinterpret_cast<const Raw4<Tin>*>(k + 4 * c + 4 * C * j);
        float qf[4], kf[4];
        widen4<Tin>(nd.q[j], qf);
        widen4<Tin>(nd.k[j], kf);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qq = fmaf(qf[e], qf[e], qq);
          kk = fmaf(kf[e], kf[e], kk);
        }
      }
      qq = e4::group_sum<C>(qq);
      kk = e4::group_sum<C>(kk);
      const IS* v = static_cast<const IS*>(a.v) + tok * a.stride_v + static_cast<int64_t>(hv) * a.V;
#pragma unroll
      for (int s = 0; s < RPT; ++s) nd.v[s] = v[rows[s] < a.V ? rows[s] : a.V - 1];
      const float2 g = gate_of(load_raw(a.a, tok * a.stride_a + hv, a.gate_dtype),
                               load_raw(a.b, tok * a.stride_b + hv, a.gate_dtype), a.gate_dtype, 1.0f, 20.0f, A,
                               dt_bias);
      nd.sc = make_float4(g.x, g.y, a.scale / sqrtf(qq + 1e-6f), 1.0f / sqrtf(kk + 1e-6f));
      settle_loads();
    }
  };

  // One node's step (:82-92): h *= exp(g); v' = (v - h k^) beta; h += k^ v'; o = h q^. The normalisation is folded:
  // h k^ = ks (h k), k^ v' = k (ks v'), o = qs (h q).
  auto advance = [&](const Node<E, RPT, Tin>& nd, float (&dv)[RPT], float (&o)[RPT], float (&kf)[E]) {
    const float decay = nd.sc.x, beta = nd.sc.y, qs = nd.sc.z, ks = nd.sc.w;
    const float dks = decay * ks;
    float qf[E];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      widen4<Tin>(nd.q[j], &qf[4 * j]);
      widen4<Tin>(nd.k[j], &kf[4 * j]);
    }
#pragma unroll
    for (int s = 0; s < RPT; ++s) {
      float hk = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) hk = fmaf(h[s][e], kf[e], hk);
      hk = e4::group_sum<C>(hk);
      dv[s] = (Tin::to_f32(nd.v[s]) - hk * dks) * beta;
      const float kdv = dv[s] * ks;
      float hq = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        h[s][e] = fmaf(kf[e], kdv, h[s][e] * decay);
        hq = fmaf(h[s][e], qf[e], hq);
      }
      o[s] = e4::group_sum<C>(hq) * qs;
    }
  };
  auto round_h = [&]() {
    if constexpr (!kPoolExact) {
#pragma unroll
      for (int s = 0; s < RPT; ++s)
#pragma unroll
        for (int e = 0; e < E; ++e) h[s][e] = e4::round_through<Tpool>(h[s][e]);
    }
  };
  // The state of node p by replaying its root path from the pool state (a parent the stack had no room for).
  auto replay = [&](int p) {
    int pv = -1, len = 0;  // lane d: the d-th ancestor-or-self of p
    for (int x = p; x >= 0 && len < 64; x = readlane(par, x)) {
      if (lane == len) pv = x;
      ++len;
    }
    load_h0();
    settle_loads();
    for (int d = len - 1; d >= 0; --d) {
      Node<E, RPT, Tin> nd;
      fetch(nd, readlane(pv, d));
      if (round && d < len - 1) round_h();
      float dv[RPT], o[RPT], kf[E];
      advance(nd, dv, o, kf);
    }
  };
  float4 (*const my_stack)[RPT * NJ][64] = stack[wave];
  float* const rec_base = a.records + (rec_idx >= 0 ? rec_idx : 0) * a.stride_records_row;

  int u = chain ? 0 : (roots != 0 ? static_cast<int>(__builtin_ctzll(roots)) : -1);
  if (u < 0) return;
  Node<E, RPT, Tin> cur, nxt;
  fetch(cur, u);
  int sp = 0;
  uint64_t unparked = 0;
  for (int it = 0; it < Tn && u >= 0; ++it) {
    int next = -1;
    bool next_first = false, next_last = false, next_root = false;
    if (chain) {
      next = u + 1 < Tn ? u + 1 : -1;
    } else {
      const uint64_t ku = readlane64(kids, u);
      if (ku != 0) {
        next = __builtin_ctzll(ku);
        next_first = true;
      } else {
        for (int x = u, hops = 0; hops < 64; ++hops) {  // a visited node's ancestors lead to a root
          const int px = readlane(par, x);
          const uint64_t above = x == 63 ? 0 : ~0ull << (x + 1);
          if (px < 0) {  // x is a root: the next root starts from the pool state
            const uint64_t nr = roots & above;
            if (nr != 0) {
              next = __builtin_ctzll(nr);
              next_root = true;
            }
            break;
          }
          const uint64_t sib = readlane64(kids, px) & above;
          if (sib != 0) {
            next = __builtin_ctzll(sib);
            next_last = (sib & (sib - 1)) == 0;
            break;
          }
          x = px;
        }
      }
    }
    if (next >= 0 && next < TS) fetch(nxt, next);

    float dv[RPT], o[RPT], kf[E];
    advance(cur, dv, o, kf);
    const int64_t t = bos + u;
    if (c == 0) {
#pragma unroll
      for (int s = 0; s < RPT; ++s) {
        if (rows[s] < a.V) {
          e4::store_scalar(a.out, t * a.stride_o + static_cast<int64_t>(hv) * a.V + rows[s], a.out_dtype, o[s]);
          if (rec_idx >= 0)
            rec_base[(static_cast<int64_t>(u) * a.HV + hv) * a.rec + rows[s]] = dv[s];
        }
      }
    }
    if (rec_idx >= 0 && blockIdx.x == 0 && wave == 0) {  // the key (normalised) and the decay, once per node
      float* kr = rec_base + (static_cast<int64_t>(u) * a.HV + hv) * a.rec + a.V;
      if (rr == 0) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) kr[4 * c + 4 * C * j + e] = kf[4 * j + e] * cur.sc.w;
      }
      if (lane == 0) kr[K] = cur.sc.x;
    }

    if (next >= 0 && !chain) {
      const uint64_t ku = readlane64(kids, u);
      if ((ku & (ku - 1)) != 0) {  // several children: park the state (as its children read it)
        if (sp < S) {
#pragma unroll
          for (int s = 0; s < RPT; ++s)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              float4 w = make_float4(h[s][4 * j], h[s][4 * j + 1], h[s][4 * j + 2], h[s][4 * j + 3]);
              if (round)
                w = make_float4(e4::round_through<Tpool>(w.x), e4::round_through<Tpool>(w.y),
                                e4::round_through<Tpool>(w.z), e4::round_through<Tpool>(w.w));
              my_stack[sp][s * NJ + j][lane] = w;
            }
          ++sp;
        } else {
          unparked |= 1ull << u;
        }
      }
      if (next_first) {
        if (round) round_h();
      } else if (next_root) {
        load_h0();
        settle_loads();
      } else {
        const int p = readlane(par, next);
        if ((unparked >> p) & 1) {
          replay(p);
          if (round) round_h();
        } else {
#pragma unroll
          for (int s = 0; s < RPT; ++s)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              const float4 w = my_stack[sp - 1][s * NJ + j][lane];
              h[s][4 * j] = w.x;
              h[s][4 * j + 1] = w.y;
              h[s][4 * j + 2] = w.z;
              h[s][4 * j + 3] = w.w;
            }
          if (next_last) --sp;
        }
      }
    }
    if (next >= 0) {
      if (next < TS)
        cur = nxt;
      else
        fetch(cur, next);
    }
    u = next;
  }
}

template <int K, int C, int RPT, int WAVES, int S, typename Tin>
int launch_records_pool(const eagle4_records_args& a, hipStream_t s) {
  constexpr int ROWS = WAVES * RPT * (64 / C);
  const dim3 grid(e4::ceil_div(a.V, ROWS), a.HV, a.N);
  if (a.state_dtype == EAGLE4_F32)
    gdn_records_walk_kernel<K, C, RPT, WAVES, S, Tin, e4::F32><<<grid, 64 * WAVES, 0, s>>>(a);
  else if (a.state_dtype == EAGLE4_BF16)
    gdn_records_walk_kernel<K, C, RPT, WAVES, S, Tin, e4::Bf16><<<grid, 64 * WAVES, 0, s>>>(a);
  else if (a.state_dtype == EAGLE4_F16)
    gdn_records_walk_kernel<K, C, RPT, WAVES, S, Tin, e4::F16><<<grid, 64 * WAVES, 0, s>>>(a);
  else
    return EAGLE4_NOT_COVERED;
  return E4_LAUNCH_STATUS();
}

template <int K, int C, int RPT, int WAVES, int S>
int launch_records(const eagle4_records_args& a, hipStream_t s) {
  if (a.in_dtype == EAGLE4_BF16) return launch_records_pool<K, C, RPT, WAVES, S, e4::Bf16>(a, s);
  if (a.in_dtype == EAGLE4_F16) return launch_records_pool<K, C, RPT, WAVES, S, e4::F16>(a, s);
  if (a.in_dtype == EAGLE4_F32) return launch_records_pool<K, C, RPT, WAVES, S, e4::F32>(a, s);
  return EAGLE4_NOT_COVERED;
}

// ---- commit ------------------------------------------------------------------------------------------------------
// 4 waves x 8 rows: one (32-row V tile, request x value head, layer) per workgroup; lane layout as in the walk.
template <int K, int C, typename Tpool>
__global__ __launch_bounds__(256) void gdn_records_commit_kernel(const eagle4_records_commit_args a) {
  constexpr int E = K / C;
  constexpr int NJ = E / 4;
  constexpr int ROWS = 4 * (64 / C);
  using PS = typename Tpool::storage;
  __shared__ int s_path[64];
  __shared__ int s_len;
  const int nh = blockIdx.y, layer = blockIdx.z;
  const int n = nh / a.HV, hv = nh % a.HV;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane % C, rr = lane / C;
  const int row = blockIdx.x * ROWS + wave * (64 / C) + rr;
  const int64_t step = e4::ld(a.commit_steps, n), slot = e4::ld(a.state_indices, n), rrow = e4::ld(a.record_indices, n);
  if (!(step >= 0 && slot >= 0 && rrow >= 0)) return;
  if (tid == 0) {  // the root path, accepted node first (:192-201)
    int node = static_cast<int>(step), len = 0;
    for (int j = 0; j < a.dmax && j < 64 && node >= 0 && node < a.dmax; ++j) {
      s_path[len++] = node;
      node = node > 0 ? static_cast<int>(e4::ld(a.parent, n, node)) : -1;
    }
    s_len = len;
  }
  __syncthreads();
  const int len = s_len;
  PS* st = static_cast<PS*>(a.state) + layer * a.stride_state_layer + slot * a.stride_state_slot +
           static_cast<int64_t>(hv) * a.V * K + static_cast<int64_t>(row < a.V ? row : 0) * K;
  const float* rec = a.records + layer * a.stride_records_layer + rrow * a.stride_records_row;
  float h[E];
#pragma unroll
  for (int j = 0; j < NJ; ++j) load4<Tpool>(st + 4 * c + 4 * C * j, &h[4 * j]);
  for (int d = 0; d < len; ++d) {
    const float* r = rec + (static_cast<int64_t>(s_path[len - 1 - d]) * a.HV + hv) * a.rec;
    const float eg = r[a.V + K];
    const float delta = r[row < a.V ? row : 0];
    if (a.round_state && d > 0) {
#pragma unroll
      for (int e = 0; e < E; ++e) h[e] = e4::round_through<Tpool>(h[e]);
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float key = r[a.V + 4 * c + 4 * C * j + e];
        h[4 * j + e] = h[4 * j + e] * eg + key * delta;
      }
    }
  }
  if (row < a.V) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) store4<Tpool>(st + 4 * c + 4 * C * j, &h[4 * j]);
  }
}

template <int K, int C>
int launch_commit(const eagle4_records_commit_args& a, hipStream_t s) {
  constexpr int ROWS = 4 * (64 / C);
  const dim3 grid(e4::ceil_div(a.V, ROWS), a.n * a.HV, a.layers);
  if (a.state_dtype == EAGLE4_F32)
    gdn_records_commit_kernel<K, C, e4::F32><<<grid, 256, 0, s>>>(a);
  else if (a.state_dtype == EAGLE4_BF16)
    gdn_records_commit_kernel<K, C, e4::Bf16><<<grid, 256, 0, s>>>(a);
  else if (a.state_dtype == EAGLE4_F16)
    gdn_records_commit_kernel<K, C, e4::F16><<<grid, 256, 0, s>>>(a);
  else
    return EAGLE4_NOT_COVERED;
  return E4_LAUNCH_STATUS();
}

}  // namespace

extern "C" int eagle4_gdn_tree_records_update(const eagle4_records_args* a, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->N == 0) return EAGLE4_OK;
  const int64_t esz = a->in_dtype == EAGLE4_F32 ? 4 : 2;
  if (a->H <= 0 || a->HV % a->H != 0 || a->V <= 0 || a->width <= 0 || a->width > 64 || a->rec < a->V + a->K + 1 ||
      !e4::is_float_dtype(a->gate_dtype) || !e4::is_float_dtype(a->out_dtype) || !e4::is_float_dtype(a->A_log_dtype) ||
      !e4::is_float_dtype(a->dt_bias_dtype) || a->query_start_loc.ptr == nullptr ||
      a->state_indices.ptr == nullptr || a->record_indices.ptr == nullptr ||
      (a->path_replay && (a->tree_paths.ptr == nullptr || a->tree_paths.dtype != EAGLE4_I32 || a->num_paths < 0)) ||
      (!a->path_replay && a->parent.ptr == nullptr) || a->stride_q % 4 || a->stride_k % 4 || a->stride_v % 4 ||
      reinterpret_cast<uintptr_t>(a->q) % (4 * esz) || reinterpret_cast<uintptr_t>(a->k) % (4 * esz) ||
      reinterpret_cast<uintptr_t>(a->v) % (4 * esz))
    return EAGLE4_NOT_COVERED;
  {
    const int st = a->path_replay ? e4replay::launch(*a, s) : e4chunk::launch(*a, s);
    if (st != EAGLE4_NOT_COVERED) return st;
  }
  switch (a->K) {
    case 8: return launch_records<8, 2, 1, 2, 4>(*a, s);
    case 16: return launch_records<16, 4, 1, 2, 4>(*a, s);
    case 32: return launch_records<32, 8, 1, 2, 4>(*a, s);
    case 64: return launch_records<64, 8, 1, 2, 4>(*a, s);
    case 128: return launch_records<128, 8, 1, 2, 4>(*a, s);
    case 256: return launch_records<256, 16, 1, 2, 4>(*a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}

extern "C" int eagle4_gdn_tree_records_commit(const eagle4_records_commit_args* a, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (a->n == 0 || a->layers == 0) return EAGLE4_OK;
  if (a->HV <= 0 || a->V <= 0 || a->dmax <= 0 || a->rec < a->V + a->K + 1 || a->commit_steps.ptr == nullptr ||
      a->state_indices.ptr == nullptr || a->record_indices.ptr == nullptr || a->parent.ptr == nullptr)
    return EAGLE4_NOT_COVERED;
  switch (a->K) {
    case 8: return launch_commit<8, 2>(*a, s);
    case 16: return launch_commit<16, 4>(*a, s);
    case 32: return launch_commit<32, 8>(*a, s);
    case 64: return launch_commit<64, 8>(*a, s);
    case 128: return launch_commit<128, 8>(*a, s);
    case 256: return launch_commit<256, 16>(*a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}
