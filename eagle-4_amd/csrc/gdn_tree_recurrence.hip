// Gated delta rule over a draft tree on gfx950, snapshot contract (kernels/gdn_tree_recurrence.py:204-359, 562-706).
//
// Roofline: HBM writes. Every node of every (request, value head) writes its whole [V, K] state snapshot (64 KB in
// fp32 at V = K = 128) and reads ~1 KB of inputs, at ~1.7 FLOP per byte. The layout is chosen for the stores:
//
//  * A workgroup owns one (V tile, request, value head); the tile's state lives in the VGPRs of its waves for the
//    whole walk, each wave owning RPT x (64 / C) rows.
//  * C adjacent lanes share a V row, each holding E = K / C state values as E/4 float4 chunks at k = 4c + 4Cj
//    (c = lane % C, j = chunk). At K = 128, C = 8: one store instruction writes 8 rows x 128 contiguous bytes, so
//    every snapshot store is whole 128-byte lines, streamed once.
//  * The K reductions (h k and h q) are C-lane butterflies; q / k norms reduce the same way.
//
// Which state a node starts from. The reference walks the rows in index order and, for every node but the root,
// reloads its parent's snapshot from the buffer it has just written (an fp32 chain child, parent = previous row,
// continues from registers instead; :318-329). Rows are parent first but otherwise in any order, so in index order
// most parents are not the row just computed and ~3/4 of the nodes reload 64 KB each. Here a request whose reloads
// are guaranteed to return the parent's own snapshot (parents precede children, every row has a real slot, no two
// rows share one, at most 64 rows) is walked depth first instead (pre-order): a node's first child continues from
// the registers, and a node with more children parks its state on a small per-wave LDS stack that its later children
// pop (LIFO: when a later child of p comes, every state pushed after p has been popped). A node's children are walked
// in increasing order of the stack entries their subtrees need, the neediest last, so two entries cover every tree
// whose nesting of multi-child nodes is at most two deep in that sense (all 16-node trees of up to 4 children per
// node in these workloads; in index order such trees overflow two entries ~1.1 times per tree).
// Parked states are what a reload would give (rounded through the snapshot dtype; exact in fp32), so the results
// are bit-identical to the index-order walk. When the stack is full a node is not parked and its later children
// reload its snapshot from HBM, as the reference does. Any other request keeps the reference's index-order walk
// with its reloads (the same wave wrote the snapshot it reads: same addresses, same lane, so no barrier is needed).
//
// The math and its order follow the walk: h *= exp(g); v' = (v - h k^) * beta; h += k^ v'; o = h q^, with beta
// rounded through b's dtype and q^ = q scale / |q|, k^ = k / |k| (1e-6 inside the square roots), normalised once per
// node in the prologue and kept in LDS as fp32.

#include "gdn_walk.h"
#include "walk_plan.h"

namespace {

using namespace e4walk;

// A node's inputs as a lane holds them: its E values of q^ and k^ (fp32), v of its RPT rows (raw), decay and beta.
template <int E, int RPT, typename IS>
struct NodeIn {
  float q[E], k[E];
  IS v[RPT];
  float decay, beta;
};

// Workgroup id -> (request, value head, V tile), the tile fastest: the workgroups of one request are adjacent, so the
// resident ones write a few requests' slot runs at a time. (Handing each XCD whole requests measured slower.)
E4_DEV void item_of(int id, int HV, int tiles, int& n, int& hv, int& tile) {
  const int G = tiles * HV;
  n = id / G;
  hv = (id % G) / tiles;
  tile = id % tiles;
}

// Workgroup: WAVES waves over consecutive V rows of one (request, value head); each wave owns RPT x (64 / C) rows.
// The request's first TS nodes are staged in LDS up front (q, k, the workgroup's v rows, and the node scalars), so the
// walk itself issues no global loads for them: a vector load in the walk would wait for the snapshot stores before it
// (loads and stores share the vmcnt counter), which serialises the walk on the store latency.
template <int K, int C, int RPT, int WAVES, int S, bool SMALL, typename Tin, typename Tsnap>
__global__ __launch_bounds__(64 * WAVES) void gdn_tree_walk_kernel(const eagle4_gdn_args a) {
  constexpr int E = K / C;
  constexpr int NJ = E / 4;
  constexpr int ROWS_WAVE = RPT * (64 / C);
  constexpr int ROWS = WAVES * ROWS_WAVE;
  constexpr int NT = 64 * WAVES;
  static_assert(E % 4 == 0 && C <= 64, "lane layout");
  using IS = typename Tin::storage;
  using SS = typename Tsnap::storage;
  constexpr int TS = sizeof(IS) == 4 ? 8 : 16;  // staged nodes
  constexpr bool kExact = sizeof(SS) == 4;      // fp32 snapshots: a reload gives the registers bit for bit
  constexpr bool kFastWalk = E <= 8;            // the depth-first walk of staged nodes has a loop of its own
  // The parked-state stack; in the prologue, before any state is parked, it holds the staged nodes' raw q and k rows.
  constexpr int kStackBytes = WAVES * S * RPT * NJ * 64 * 16;
  constexpr int kRawBytes = 2 * TS * K * static_cast<int>(sizeof(IS));
  __shared__ __align__(16) char s_stack[kStackBytes > kRawBytes ? kStackBytes : kRawBytes];
  __shared__ __align__(16) float s_q[TS][K];  // q^ and k^ of the staged nodes
  __shared__ __align__(16) float s_k[TS][K];
  __shared__ IS s_v[TS][ROWS];
  __shared__ float4 s_sc[TS];  // decay, beta, scale / |q|, 1 / |k|
  __shared__ __align__(16) float s_out[TS][ROWS];  // the staged nodes' outputs, stored in one pass after the walk
  auto& s_qr = *reinterpret_cast<IS(*)[TS][K]>(s_stack);
  auto& s_kr = *reinterpret_cast<IS(*)[TS][K]>(s_stack + TS * K * sizeof(IS));
  // The walk plan's scratch while wave 0 builds it and hands it over: in s_out, first written by the walk itself,
  // where it fits (16-bit inputs at 32 rows per workgroup), else LDS of its own; s_q stays free, so the staged rows'
  // norms write q^ and k^ in the same pass.
  constexpr bool kPlanInOut = sizeof(float) * TS * ROWS >= sizeof(PlanScratch);
  __shared__ __align__(16) char s_plan_own[kPlanInOut ? 16 : sizeof(PlanScratch)];
  PlanScratch& ps = *reinterpret_cast<PlanScratch*>(kPlanInOut ? reinterpret_cast<char*>(&s_out[0][0]) : s_plan_own);

  int n, hv, tile;
  item_of(blockIdx.x, a.HV, (a.V + ROWS - 1) / ROWS, n, hv, tile);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int c = lane % C, rr = lane / C;
  const int ih = hv / (a.HV / a.H);
  const int row0 = tile * ROWS;
  int rows[RPT], lrow[RPT];
#pragma unroll
  for (int s = 0; s < RPT; ++s) {
    lrow[s] = wave * ROWS_WAVE + s * (64 / C) + rr;
    rows[s] = row0 + lrow[s];
  }

  if (a.publish != nullptr && tile == 0 && hv == 0) {  // _publish_slot_table (:188-200)
    for (int i = tid; i < a.num_slot_cols; i += NT)
      a.publish[n * a.stride_publish + i] = static_cast<int32_t>(e4::ld(a.snap_indices, n, i));
  }
  // The prologue issues every load before its first wait: the request's tables, the plan tables (parents, slots),
  // the initial state, the staged nodes' inputs; the plan is computed while the last of them are in flight.
  const bool has_acc = a.num_accepted.ptr != nullptr;
  const int64_t bos = uni64(e4::ld(a.cu_seqlens, n));
  const int64_t eos = uni64(e4::ld(a.cu_seqlens, n + 1));
  const int64_t cache_idx = uni64(e4::ld(a.snap_indices, n, 0));  // the request's scratch row (per-row slots: row 0's)
  const int64_t acc_raw = uni64(e4::ld(has_acc ? a.num_accepted : a.cu_seqlens, n));  // loaded either way: no branch
  const int64_t nacc = has_acc ? acc_raw : 1;
  const uint32_t A_raw = load_raw(a.A_log, hv, a.A_log_dtype);
  const uint32_t dt_raw = load_raw(a.dt_bias, hv, a.dt_bias_dtype);
  const int T = static_cast<int>(eos - bos);
  // A launch whose snapshots outgrow the last-level cache (MI355X: 256 MB) stores them nontemporally: regular stores
  // leave a cache's worth of dirty lines that the next kernel's reads pay to write back (a 512 MB stream: 13 us
  // faster to store, 39 us slower for the kernel after it). The launch's bytes from the grid and this request's nodes.
  // The small grids (SMALL) store nontemporally too: their walk is latency-bound and its regular stores' dirty L2
  // lines are written back before the kernel counts as finished (batch 1: 13.0 -> 11.8 us, batch 2: 16.6 -> 15.9;
  // batches 4 and 8, on the 8-lane form, are 5-7 % slower with nontemporal stores).
  const bool snap_nt =
      SMALL || static_cast<int64_t>(gridDim.x) * ROWS * K * static_cast<int64_t>(sizeof(SS)) * T > (256ll << 20);
  if (T <= 0) return;

  // Lane i holds row i's parent and slot (rows of at most 64-row requests).
  int par = 0;
  int64_t my_slot = cache_idx;
  if (T <= 64 && lane < T) {
    par = static_cast<int>(e4::ld(a.parents, n, lane));
    if (a.row_slots) my_slot = e4::ld(a.snap_indices, n, lane);
  }
  // the initial state (:284-296); with num_accepted its slot is in column num_accepted - 1
  const int64_t idx = uni64(e4::ld(a.h0_indices, n, nacc - 1));
  const int64_t head_off = static_cast<int64_t>(hv) * a.V * K;
  float h[RPT][E];
  u32x4 h0raw[RPT][NJ];
#pragma unroll
  for (int s = 0; s < RPT; ++s)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      h0raw[s][j] = u32x4{0u, 0u, 0u, 0u};  // zero bits: +0.0 in every dtype
      if (idx > a.pad_slot_id && rows[s] < a.V)
        load_state_raw(a.h0_source, idx * a.stride_h0_source + head_off + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j,
                       a.h0_dtype, h0raw[s][j]);
    }
  const int ts = T < TS ? T : TS;
  // Waves 1 .. WAVES - 1 stage the nodes while wave 0 builds the walk plan, so wave 0 goes from its plan straight to
  // the barrier (batch 1: the plan is the prologue's longest path)
  static_assert(WAVES >= 2, "a plan wave and staging waves");
  Staging<Tin, K, TS, ROWS, NT - 64> stg;
  const NodeSrc src{a.q, a.k, a.v, a.a, a.b, a.stride_q, a.stride_k, a.stride_v, a.stride_a, a.stride_b,
                    a.gate_dtype, ih, hv, a.V};
  if (wave > 0) stg.issue(src, bos, ts, row0, tid - 64);

  // The walk plan (walk_plan.h), built by wave 0 and read by every wave after the staging barrier. Depth first needs
  // reloads that return the parent's own snapshot: parents before children, every row a real slot, no two rows one.
  // Children go in increasing (need, index), except with 16-bit snapshots and the chain-child rule, where a chain
  // child must be the first child (it continues unrounded from the registers), so that case keeps the index order,
  // as do the small grids (SMALL).
  if (wave == 0) {
    bool ok = T <= 64 && (a.row_slots ? true : (cache_idx > a.pad_slot_id && a.stride_snap_row != 0));
    if (ok) {
      bool bad = lane < T && ((lane > 0 && (par < 0 || par >= lane)) || my_slot <= a.pad_slot_id);
      if (a.row_slots) bad = bad || slot_repeats(static_cast<uint64_t>(my_slot), lane, T);
      ok = __ballot(bad) == 0;
    }
    ps.plan[lane] = ok ? build_plan(ps, lane, T, par, !SMALL && (kExact || !a.skip_chain_reload)) : kNoNext;
    if (lane == 0) ps.dfs = ok ? 1 : 0;
  }

  // ---- staging: q, k, v and the node scalars of nodes [0, ts) into LDS --------------------------------------------
  const float A = -expf(widen_raw(A_raw, a.A_log_dtype));
  const float dt_bias = widen_raw(dt_raw, a.dt_bias_dtype);
  if (wave > 0)
    stg.commit(s_qr, s_kr, s_v, s_sc, ts, tid - 64, a.gate_dtype, a.softplus_beta, a.softplus_threshold, A, dt_bias);
#pragma unroll
  for (int s = 0; s < RPT; ++s)
#pragma unroll
    for (int j = 0; j < NJ; ++j) widen_state_raw(h0raw[s][j], a.h0_dtype, &h[s][4 * j]);
  __syncthreads();
  const int plan = ps.plan[lane];  // read before the walk writes s_out (after the next barrier)
  const bool dfs = ps.dfs != 0;
  // L2 norms over K (:143-151) and q^, k^ (read by every node of the walk) in one pass
  stage_norms<Tin, K, TS, NT>(s_qr, s_kr, s_sc, ts, tid, a.scale, s_q, s_k);
  __syncthreads();  // the raw rows' space becomes the stack

  settle_loads();  // the initial state and the plan tables
  // lane u: the element offset of row u's snapshot slot (-1: a pad slot, never written), so that a node's store
  // address is one readlane and an add
  const int64_t my_off = my_slot > a.pad_slot_id ? my_slot * a.stride_snap_slot + lane * a.stride_snap_row : -1;
  // A node's inputs: staged nodes from LDS, later ones (T > TS) from global memory with their scalars computed here.
  auto fetch_staged = [&](NodeIn<E, RPT, IS>& nd, int u) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float4 q4 = *reinterpret_cast<const float4*>(&s_q[u][4 * c + 4 * C * j]);
      const float4 k4 = *reinterpret_cast<const float4*>(&s_k[u][4 * c + 4 * C * j]);
      nd.q[4 * j] = q4.x, nd.q[4 * j + 1] = q4.y, nd.q[4 * j + 2] = q4.z, nd.q[4 * j + 3] = q4.w;
      nd.k[4 * j] = k4.x, nd.k[4 * j + 1] = k4.y, nd.k[4 * j + 2] = k4.z, nd.k[4 * j + 3] = k4.w;
    }
#pragma unroll
    for (int s = 0; s < RPT; ++s) nd.v[s] = s_v[u][lrow[s]];
    const float4 sc = s_sc[u];
    nd.decay = sc.x;
    nd.beta = sc.y;
  };
  auto fetch = [&](NodeIn<E, RPT, IS>& nd, int u) {
    if (u < TS) {
      fetch_staged(nd, u);
    } else {
      const int64_t tok = bos + u;
      const IS* q = static_cast<const IS*>(a.q) + tok * a.stride_q + static_cast<int64_t>(ih) * K;
      const IS* kp = static_cast<const IS*>(a.k) + tok * a.stride_k + static_cast<int64_t>(ih) * K;
      Raw4<Tin> qr[NJ], kr[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        qr[j] = *reinterpret_cast<const Raw4<Tin>*>(q + 4 * c + 4 * C * j);
        kr[j] = *reinterpret_cast<const Raw4<Tin>*>(kp + 4 * c + 4 * C * j);
      }
      const IS* v = static_cast<const IS*>(a.v) + tok * a.stride_v + static_cast<int64_t>(hv) * a.V;
#pragma unroll
      for (int s = 0; s < RPT; ++s) nd.v[s] = v[rows[s] < a.V ? rows[s] : a.V - 1];
      const uint32_t ga = load_raw(a.a, tok * a.stride_a + hv, a.gate_dtype);
      const uint32_t gb = load_raw(a.b, tok * a.stride_b + hv, a.gate_dtype);
      settle_loads();
      float qq = 0.f, kk = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        widen4<Tin>(qr[j], &nd.q[4 * j]);
        widen4<Tin>(kr[j], &nd.k[4 * j]);
      }
#pragma unroll
      for (int e = 0; e < E; ++e) {
        qq = fmaf(nd.q[e], nd.q[e], qq);
        kk = fmaf(nd.k[e], nd.k[e], kk);
      }
      const float qs = a.scale / sqrtf(e4::group_sum<C>(qq) + 1e-6f);
      const float ks = 1.0f / sqrtf(e4::group_sum<C>(kk) + 1e-6f);
#pragma unroll
      for (int e = 0; e < E; ++e) {
        nd.q[e] *= qs;
        nd.k[e] *= ks;
      }
      const float2 g = gate_of(ga, gb, a.gate_dtype, a.softplus_beta, a.softplus_threshold, A, dt_bias);
      nd.decay = g.x;
      nd.beta = g.y;
    }
  };

  SS* snap = static_cast<SS*>(a.snap);

  // a node's snapshot in the buffer (slot, row)
  auto snap_at = [&](int64_t slot_of, int row) {
    return snap + slot_of * a.stride_snap_slot + static_cast<int64_t>(row) * a.stride_snap_row + head_off;
  };
  auto reload = [&](const SS* src) {
#pragma unroll
    for (int s = 0; s < RPT; ++s)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (rows[s] < a.V) load4<Tsnap>(src + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j, &h[s][4 * j]);
    settle_loads();
  };
  float4 (*const my_stack)[RPT * NJ][64] = reinterpret_cast<float4 (*)[S][RPT * NJ][64]>(s_stack)[wave];
  const bool full_tile = row0 + ROWS <= a.V;  // every row of the tile exists: stores need no row predicate

  // the delta rule step (:167-185): h *= decay; v' = (v - h k^) beta; h += k^ v'; o = h q^
  auto delta_step = [&](const NodeIn<E, RPT, IS>& nd, float (&o)[RPT]) {
    const float decay = nd.decay, beta = nd.beta;
#pragma unroll
    for (int s = 0; s < RPT; ++s) {
      float hk = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) hk = fmaf(h[s][e], nd.k[e], hk);
      hk = e4::group_sum<C>(hk);
      const float dv = (Tin::to_f32(nd.v[s]) - hk * decay) * beta;
      float hq = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        h[s][e] = fmaf(nd.k[e], dv, h[s][e] * decay);
        hq = fmaf(h[s][e], nd.q[e], hq);
      }
      o[s] = e4::group_sum<C>(hq);
    }
  };
  // a node's snapshot from the registers, to element offset off of the buffer (a real slot)
  auto store_snap = [&](int64_t off) {
    SS* dst = snap + off + head_off;
    if (full_tile && snap_nt) {
      const __amdgpu_buffer_rsrc_t r = e4walk::buffer_rsrc(dst, a.V * K * static_cast<int>(sizeof(SS)));
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int s = 0; s < RPT; ++s)
          e4walk::store4_buf<Tsnap, 2>(r, (rows[s] * K + 4 * c + 4 * C * j) * static_cast<int>(sizeof(SS)), &h[s][4 * j]);
    } else if (full_tile) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int s = 0; s < RPT; ++s)
          store4<Tsnap>(dst + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j, &h[s][4 * j]);
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int s = 0; s < RPT; ++s)
          if (rows[s] < a.V) store4<Tsnap>(dst + static_cast<int64_t>(rows[s]) * K + 4 * c + 4 * C * j, &h[s][4 * j]);
    }
  };
  // The state the node after u starts from, depth first (pl: u's plan): park u's state when it has several children;
  // a first child continues from the registers (rounded through the snapshot dtype, as a reload would give it); a
  // later child pops its parent's parked state, or reloads the parent's snapshot when the stack was full.
  int sp = 0;
  uint64_t unparked = 0;  // nodes with several children that found the stack full
  auto dfs_hand_over = [&](int u, int next, int pl) {
    if ((pl & kPlanMulti) != 0) {
      if (sp < S) {
#pragma unroll
        for (int s = 0; s < RPT; ++s)
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            float4 w = make_float4(h[s][4 * j], h[s][4 * j + 1], h[s][4 * j + 2], h[s][4 * j + 3]);
            if constexpr (!kExact)
              w = make_float4(e4::round_through<Tsnap>(w.x), e4::round_through<Tsnap>(w.y),
                              e4::round_through<Tsnap>(w.z), e4::round_through<Tsnap>(w.w));
            my_stack[sp][s * NJ + j][lane] = w;
          }
        ++sp;
      } else {
        unparked |= 1ull << u;
      }
    }
    if ((pl & kPlanFirst) != 0) {
      if constexpr (!kExact) {
        if (!(a.skip_chain_reload && next == u + 1)) {  // an fp32 chain child keeps the registers
#pragma unroll
          for (int s = 0; s < RPT; ++s)
#pragma unroll
            for (int e = 0; e < E; ++e) h[s][e] = e4::round_through<Tsnap>(h[s][e]);
        }
      }
    } else {
      const int p = readlane(par, next);
      if ((unparked >> p) & 1) {
        const int64_t pslot = a.row_slots ? static_cast<int64_t>(readlane64(static_cast<uint64_t>(my_slot), p)) : cache_idx;
        reload(snap_at(pslot, p));
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
        if ((pl & kPlanLast) != 0) --sp;
      }
    }
  };

  NodeIn<E, RPT, IS> cur, nxt;
  // (lanes holding at most 8 state values per row: the latency-bound small grids at K = 128 and the small heads; with
  // 16 values the second input set and state copy would cost the store-bound large grids a wave per SIMD)
  if (kFastWalk && dfs && T <= TS && full_tile) {
    // The common request: depth first, every node staged, every row of the tile present, so a node decides nothing
    // but what its plan word says. Two nodes per trip with the two input sets' roles swapped: the next node's inputs
    // are read from LDS into the idle set ahead of their use and never copied.
    auto step = [&](int& u, const NodeIn<E, RPT, IS>& cu, NodeIn<E, RPT, IS>& nx) {
      const int pl = readlane(plan, u);
      int next = plan_next(pl);
      if (next >= T) next = -1;  // (never: plan rows are the request's)
      // This node's inputs (read one node ago) have landed by now: settling them before the next node's reads are
      // issued lets those stay in flight through this node's math (LDS returns in order, so a wait placed after them
      // would wait for them too). The reads are unconditional (the last node reads row 0 again), so no path joins
      // with a different count of reads in flight.
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      fetch_staged(nx, next >= 0 ? next : 0);
      float o[RPT];
      delta_step(cu, o);
#pragma unroll
      for (int s = 0; s < RPT; ++s) s_out[u][lrow[s]] = o[s];
      store_snap(static_cast<int64_t>(readlane64(static_cast<uint64_t>(my_off), u)));
      if (next >= 0) dfs_hand_over(u, next, pl);
      u = next;
    };
    fetch_staged(cur, 0);
    int u = 0;
    for (int it = 0;;) {  // T nodes: the plan's last node has no next (and the count bounds a malformed plan)
      step(u, cur, nxt);
      if (u < 0 || ++it >= T) break;
      step(u, nxt, cur);
      if (u < 0 || ++it >= T) break;
    }
  } else {
    fetch(cur, 0);
    int u = 0;
    for (int it = 0; it < T; ++it) {
      // the next node and where its state comes from
      int next = -1, pl = 0;
      if (dfs) {
        pl = readlane(plan, u);
        next = plan_next(pl);
        if (next >= T) next = -1;  // (never: plan rows are the request's)
      } else if (u + 1 < T) {
        next = u + 1;
      }
      if (next >= 0 && next < TS) fetch(nxt, next);  // staged: LDS reads only, ahead of their use

      float o[RPT];
      delta_step(cur, o);
      const int64_t t = bos + u;
      if (u < TS) {  // every lane of a row holds its sum: all write it (no lane branch in the walk)
#pragma unroll
        for (int s = 0; s < RPT; ++s) s_out[u][lrow[s]] = o[s];
      } else if (c == 0) {
#pragma unroll
        for (int s = 0; s < RPT; ++s)
          if (rows[s] < a.V) e4::store_scalar(a.out, t * a.stride_o + static_cast<int64_t>(hv) * a.V + rows[s], a.out_dtype, o[s]);
      }
      int64_t off = -1;  // the node's snapshot, elements from snap before head_off
      if (a.row_slots && dfs) {
        off = static_cast<int64_t>(readlane64(static_cast<uint64_t>(my_off), u));
      } else {
        int64_t slot = cache_idx;
        if (a.row_slots) {
          slot = uni64(e4::ld(a.snap_indices, n, u));
          settle_loads();
        }
        if (slot > a.pad_slot_id) off = slot * a.stride_snap_slot + static_cast<int64_t>(u) * a.stride_snap_row;
      }
      if (off >= 0) store_snap(off);

      // the state the next node starts from
      if (next >= 0) {
        if (dfs) {
          dfs_hand_over(u, next, pl);
        } else {
          // the reference's rule (:312-329)
          const int p = uni(static_cast<int>(e4::ld(a.parents, n, next)));
          const int64_t pslot = a.row_slots && p >= 0 ? uni64(e4::ld(a.snap_indices, n, p)) : cache_idx;
          bool re = p >= 0 && pslot > a.pad_slot_id;
          if (a.skip_chain_reload) re = re && p != next - 1;
          if (re) reload(snap_at(pslot, p));
        }
        if (next < TS)
          cur = nxt;
        else
          fetch(cur, next);
      }
      u = next;
    }
  }
  // the staged nodes' outputs: each wave its own rows (written above by this wave; in-order LDS), node-major
  for (int i = lane; i < ts * ROWS_WAVE; i += 64) {
    const int t = i / ROWS_WAVE, lr = wave * ROWS_WAVE + i % ROWS_WAVE, row = row0 + lr;
    if (row < a.V)
      e4::store_scalar(a.out, (bos + t) * a.stride_o + static_cast<int64_t>(hv) * a.V + row, a.out_dtype, s_out[t][lr]);
  }
}

template <int K, int C, int RPT, int WAVES, int S, bool SMALL, typename Tin>
int launch_snap(const eagle4_gdn_args& a, hipStream_t s) {
  constexpr int ROWS = WAVES * RPT * (64 / C);
  const dim3 grid(e4::ceil_div(a.V, ROWS) * a.HV * a.N);
  if (a.snap_dtype == EAGLE4_F32)
    gdn_tree_walk_kernel<K, C, RPT, WAVES, S, SMALL, Tin, e4::F32><<<grid, 64 * WAVES, 0, s>>>(a);
  else if (a.snap_dtype == EAGLE4_BF16)
    gdn_tree_walk_kernel<K, C, RPT, WAVES, S, SMALL, Tin, e4::Bf16><<<grid, 64 * WAVES, 0, s>>>(a);
  else if (a.snap_dtype == EAGLE4_F16)
    gdn_tree_walk_kernel<K, C, RPT, WAVES, S, SMALL, Tin, e4::F16><<<grid, 64 * WAVES, 0, s>>>(a);
  else
    return EAGLE4_NOT_COVERED;
  return E4_LAUNCH_STATUS();
}

template <int K, int C, int RPT, int WAVES, int S, bool SMALL = false>
int launch_in(const eagle4_gdn_args& a, hipStream_t s) {
  if (a.in_dtype == EAGLE4_BF16) return launch_snap<K, C, RPT, WAVES, S, SMALL, e4::Bf16>(a, s);
  if (a.in_dtype == EAGLE4_F16) return launch_snap<K, C, RPT, WAVES, S, SMALL, e4::F16>(a, s);
  if (a.in_dtype == EAGLE4_F32) return launch_snap<K, C, RPT, WAVES, S, SMALL, e4::F32>(a, s);
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
  // q, k, v rows are read in 4-element chunks
  const int64_t esz = a->in_dtype == EAGLE4_F32 ? 4 : 2;
  if (a->stride_q % 4 || a->stride_k % 4 || a->stride_v % 4 || reinterpret_cast<uintptr_t>(a->q) % (4 * esz) ||
      reinterpret_cast<uintptr_t>(a->k) % (4 * esz) || reinterpret_cast<uintptr_t>(a->v) % (4 * esz))
    return EAGLE4_NOT_COVERED;
  // 4 waves per workgroup; up to 16 state values per lane and stack slot
  switch (a->K) {
    case 8: return launch_in<8, 2, 1, 4, 4>(*a, s);
    case 16: return launch_in<16, 4, 1, 4, 4>(*a, s);
    case 32: return launch_in<32, 8, 1, 4, 4>(*a, s);
    case 64: return launch_in<64, 8, 1, 4, 4>(*a, s);
    case 128: {
      // 8 lanes per row, 32 rows per workgroup; a grid that leaves CUs idle that way (gfx950 parts have 256; batch 1-2
      // at 32 value heads) takes 16 lanes per row instead: each node's dependent chains (the h k and h q sums over a
      // lane's K values) halve and the grid doubles. Batch 1 24.3 -> 21.7 us, batch 2 25.2 -> 24.3 us; from batch 4
      // up (4 x 32 x 4 workgroups) the 8-lane form is faster (batch 64: 375 against 396 us).
      const int64_t groups8 = e4::ceil_div(a->V, 32) * static_cast<int64_t>(a->HV) * a->N;
      // These grids' walks are latency-bound and the need order is the plan's longest part (depths by pointer
      // jumping, then a pass per tree level): they walk children in index order and park up to four states instead
      // of two, enough for the nesting of index order in drafted trees (a parent beyond them reloads its snapshot),
      // and store their snapshots nontemporally.
      if (groups8 <= 256) return launch_in<128, 16, 1, 4, 4, true>(*a, s);
      return launch_in<128, 8, 1, 4, 2>(*a, s);
    }
    case 256: return launch_in<256, 16, 1, 4, 2>(*a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}
