// Mamba2 tree verify (kernels/mamba2_tree.py): the selective state update of every tree node, each continuing from
// its parent, on gfx950.
//
// One workgroup per (block of head dims, request, head). The (head_dim x dstate) state is spread over the workgroup:
// LPR = dstate / 16 lanes share a head-dim row m, each holding 16 fp32 state elements as four 4-element chunks
// c = lane_in_row + LPR j (so a row's lanes write one contiguous run per store), a wave holds 64 / LPR rows and the
// four waves 256 / LPR. Every node updates the state in registers (exp(A dt) decay, dt B x input), stores it to its
// slot and reduces C . state over the row's lanes (xor shuffles). The walk is store-bound: every node writes
// head_dim x dstate state elements.
//
// Which state a node starts from. The reference walks the rows in index order; a row whose parent is the previous
// row continues from the registers, any other reloads its parent's stored state (rounded through the pool dtype;
// zeros for a pad slot). Here a request whose reloads are guaranteed to return the parent's own stored state (parents
// precede children, every row has a real slot, no two rows share one, at most 64 rows) is walked depth first: a
// node's first child continues from the registers (rounded through the pool dtype unless it is the chain child, as
// the reference's reload would round it), and a node with more children parks its state, rounded as a reload would
// give it, on a per-wave LDS stack of two entries that its later children pop. With an fp32 pool the children are
// walked in increasing order of the stack entries their subtrees need (Sethi-Ullman numbering, the neediest last),
// so two entries cover the trees; a 16-bit pool keeps the index order among children (its chain child, the lowest
// index, must come first to continue unrounded). When the stack is full the later children reload from HBM as the
// reference does. Any other request keeps the reference's index-order walk with its reloads (each lane reads back
// only elements it wrote itself, so no barrier is needed; :56-61 of the reference's walk).
//
// No load waits behind stores: gfx950 counts loads and stores in one vmcnt, so a global load inside the node loop
// would wait for the snapshot stores before it. The first TS nodes' B, C (fp32), x rows and (dt, exp(A dt)) are staged
// in LDS before the walk; later nodes and the rare reloads settle their own loads.

#include "gdn_walk.h"
#include "walk_plan.h"

namespace {

using e4walk::readlane;
using e4walk::readlane64;
using e4walk::settle_loads;
using e4walk::uni;
using e4walk::uni64;
using e4walk::PlanScratch;
using e4walk::build_plan;
using e4walk::kNoNext;
using e4walk::kPlanFirst;
using e4walk::kPlanLast;
using e4walk::kPlanMulti;
using e4walk::plan_next;
using e4walk::slot_repeats;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int NT = 256;
constexpr int kStack = 2;  // parked states per wave

template <typename S>
E4_DEV f32x4 load4(const typename S::storage* p) {
  if constexpr (sizeof(typename S::storage) == 4) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    const u32x2 r = *reinterpret_cast<const u32x2*>(p);
    return f32x4{S::to_f32(static_cast<uint16_t>(r.x & 0xffff)), S::to_f32(static_cast<uint16_t>(r.x >> 16)),
                 S::to_f32(static_cast<uint16_t>(r.y & 0xffff)), S::to_f32(static_cast<uint16_t>(r.y >> 16))};
  }
}

template <typename S>
E4_DEV void store4(typename S::storage* p, f32x4 v) {
  if constexpr (sizeof(typename S::storage) == 4) {
    *reinterpret_cast<f32x4*>(p) = v;
  } else {
    const uint32_t lo = S::from_f32(v.x) | (static_cast<uint32_t>(S::from_f32(v.y)) << 16);
    const uint32_t hi = S::from_f32(v.z) | (static_cast<uint32_t>(S::from_f32(v.w)) << 16);
    *reinterpret_cast<u32x2*>(p) = u32x2{lo, hi};
  }
}

// four elements of B or C (in_dtype) as fp32
E4_DEV f32x4 load_in4(const void* p, int64_t i, int dtype) {
  if (dtype == EAGLE4_F32) return *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i);
  if (dtype == EAGLE4_BF16) return load4<e4::Bf16>(static_cast<const uint16_t*>(p) + i);
  return load4<e4::F16>(static_cast<const uint16_t*>(p) + i);
}

// softplus as the reference writes it (:38-39): log(exp(dt) + 1) up to 20, dt above
E4_DEV float softplus(float dt) { return dt <= 20.f ? logf(expf(dt) + 1.f) : dt; }

template <int LPR, typename S>
__global__ __launch_bounds__(NT) void mamba2_tree_kernel(const eagle4_mamba2_args a) {
  using SS = typename S::storage;
  constexpr int ROWS = NT / LPR;           // head-dim rows per workgroup
  constexpr int DS = 16 * LPR;             // dstate
  constexpr int TS = DS >= 256 ? 8 : 16;   // staged nodes
  constexpr bool kExact = sizeof(SS) == 4; // fp32 pool: a reload gives the registers bit for bit
  __shared__ __align__(16) f32x4 s_stack[NT / 64][kStack][4][64];
  __shared__ __align__(16) float s_B[TS][DS];
  __shared__ __align__(16) float s_C[TS][DS];
  __shared__ float s_x[TS][ROWS];
  __shared__ float2 s_g[TS];  // a staged node's (dt, exp(A dt))
  __shared__ PlanScratch s_plan;  // the walk plan, built by wave 0

  const int b = blockIdx.y, h = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane % LPR;
  const int row0 = blockIdx.x * ROWS;
  const int lrow = wave * (64 / LPR) + lane / LPR;  // the lane's row within the workgroup
  const int m = row0 + lrow;
  const bool mok = m < a.head_dim;
  // the request's table entries, loaded together (no branch on a table's dtype)
  const bool has_acc = a.num_accepted.ptr != nullptr;
  const int64_t bos = uni64(e4::ld(a.query_start_loc, b));
  const int T = static_cast<int>(uni64(e4::ld(a.query_start_loc, b + 1)) - bos);
  const int64_t acc = uni64(e4::ld(has_acc ? a.num_accepted : a.query_start_loc, b));  // loaded either way
  if (T <= 0) return;
  // A launch whose stored states outgrow the last-level cache (MI355X: 256 MB) stores them nontemporally: regular
  // stores leave a cache's worth of dirty lines that the next kernel's reads pay to write back. The launch's bytes from
  // the grid and this request's nodes.
  const bool state_nt = static_cast<int64_t>(gridDim.x) * gridDim.y * gridDim.z * T * ROWS * DS *
                            static_cast<int64_t>(sizeof(SS)) > (256ll << 20);
  const int g = h / (a.heads / a.groups);
  const int64_t pad = a.pad_slot_id;
  SS* const hstate = static_cast<SS*>(a.state) + h * a.stride_state_head + static_cast<int64_t>(m) * a.stride_state_dim;
  const float A = a.A[h];
  const float Dh = a.D != nullptr ? e4::load_scalar(a.D, h, a.param_dtype) : 0.f;
  const float dtb = a.dt_bias != nullptr ? e4::load_scalar(a.dt_bias, h, a.param_dtype) : 0.f;

  f32x4 st[4];
  auto load_slot = [&](int64_t slot) {  // a stored state (zeros for the pad slot), this lane's elements
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 4 * (lr + LPR * j);
      st[j] = (slot != pad && mok) ? load4<S>(hstate + slot * a.stride_state_slot + n) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  // the prologue issues its loads before its first wait: the start state, the plan tables, the staged nodes
  const int64_t init_row = has_acc ? (acc - 1 > 0 ? acc - 1 : 0) : 0;
  int par = -1;
  int64_t my_slot = pad;
  if (lane < T && lane < 64) {
    par = static_cast<int>(e4::ld(a.parents, b, lane));
    my_slot = e4::ld(a.slots, b, lane);
  }
  load_slot(uni64(e4::ld(a.slots, b, init_row)));
  const int ts = T < TS ? T : TS;
  for (int i = tid; i < ts * (DS / 4); i += NT) {  // B and C of the staged nodes, fp32
    const int t = i / (DS / 4), n = 4 * (i % (DS / 4));
    const int64_t tok = bos + t;
    *reinterpret_cast<f32x4*>(&s_B[t][n]) = load_in4(a.B, tok * a.stride_B_tok + g * a.stride_B_group + n, a.in_dtype);
    *reinterpret_cast<f32x4*>(&s_C[t][n]) = load_in4(a.C, tok * a.stride_C_tok + g * a.stride_C_group + n, a.in_dtype);
  }
  for (int i = tid; i < ts * ROWS; i += NT) {  // x of the workgroup's rows
    const int t = i / ROWS, r = i % ROWS;
    s_x[t][r] = row0 + r < a.head_dim
                    ? e4::load_scalar(a.x, (bos + t) * a.stride_x_tok + h * a.stride_x_head + row0 + r, a.in_dtype)
                    : 0.f;
  }
  if (tid < ts) {
    float dt = e4::load_scalar(a.dt, (bos + tid) * a.stride_dt_tok + h * a.stride_dt_head, a.dt_dtype) + dtb;
    if (a.dt_softplus) dt = softplus(dt);
    s_g[tid] = make_float2(dt, exp2f(1.4426950408889634f * (A * dt)));
  }

  // The walk plan (walk_plan.h), built by wave 0 and read by every wave after the staging barrier: depth first when
  // the reloads are guaranteed to return the parent's own state; children in increasing (need, index) with an fp32
  // pool, by index with a 16-bit one.
  if (wave == 0) {
    bool ok = T <= 64;
    if (ok) {
      bool bad = lane < T && ((lane > 0 && (par < 0 || par >= lane)) || my_slot == pad);
      bad = bad || slot_repeats(static_cast<uint64_t>(my_slot), lane, T);
      ok = __ballot(bad) == 0;
    }
    s_plan.plan[lane] = ok ? build_plan(s_plan, lane, T, par, kExact) : kNoNext;
    if (lane == 0) s_plan.dfs = ok ? 1 : 0;
  }
  settle_loads();
  __syncthreads();  // the staged nodes and the plan
  const int plan = s_plan.plan[lane];
  const bool dfs = s_plan.dfs != 0;

  // node t's (dt, exp(A dt)), x and B / C chunks: staged, or (past TS) from global memory, settled here
  auto node_in = [&](int t, float2& gd, float& x, f32x4 (&Bv)[4], f32x4 (&Cv)[4]) {
    if (t < TS) {
      gd = s_g[t];
      x = s_x[t][lrow];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = 4 * (lr + LPR * j);
        Bv[j] = *reinterpret_cast<const f32x4*>(&s_B[t][n]);
        Cv[j] = *reinterpret_cast<const f32x4*>(&s_C[t][n]);
      }
    } else {
      const int64_t tok = bos + t;
      float dt = e4::load_scalar(a.dt, tok * a.stride_dt_tok + h * a.stride_dt_head, a.dt_dtype) + dtb;
      x = mok ? e4::load_scalar(a.x, tok * a.stride_x_tok + h * a.stride_x_head + m, a.in_dtype) : 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = 4 * (lr + LPR * j);
        Bv[j] = load_in4(a.B, tok * a.stride_B_tok + g * a.stride_B_group + n, a.in_dtype);
        Cv[j] = load_in4(a.C, tok * a.stride_C_tok + g * a.stride_C_group + n, a.in_dtype);
      }
      settle_loads();
      if (a.dt_softplus) dt = softplus(dt);
      gd = make_float2(dt, exp2f(1.4426950408889634f * (A * dt)));
    }
  };

  f32x4 (*const my_stack)[4][64] = s_stack[wave];
  int u = 0, sp = 0;
  uint64_t unparked = 0;  // nodes with several children that found the stack full
  for (int it = 0; it < T; ++it) {
    // the next node
    int next = -1, pl = 0;
    if (dfs) {
      pl = readlane(plan, u);
      next = plan_next(pl);
      if (next >= T) next = -1;  // (never: plan rows are the request's)
    } else if (u + 1 < T) {
      next = u + 1;
    }
    const bool next_first = (pl & kPlanFirst) != 0, next_last = (pl & kPlanLast) != 0;

    // the selective state update of row u (:62-80): s = s exp(A dt) + dt B x; out = C . s + D x
    float2 gd;
    float x;
    f32x4 Bv[4], Cv[4];
    node_in(u, gd, x, Bv, Cv);
    const int64_t tok = bos + u;
    const int64_t row_slot = dfs ? static_cast<int64_t>(readlane64(static_cast<uint64_t>(my_slot), u))
                                 : uni64(e4::ld(a.slots, b, u));
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 4 * (lr + LPR * j);
      st[j] = st[j] * gd.y + (Bv[j] * gd.x) * x;
      if (row_slot != pad && mok) {
        if (state_nt) {  // buffer stores: the nt policy is an immediate the compiler cannot merge away
          SS* const head = static_cast<SS*>(a.state) + h * a.stride_state_head + row_slot * a.stride_state_slot;
          const int bytes = static_cast<int>(((a.head_dim - 1) * a.stride_state_dim + DS) * sizeof(SS));
          const float w[4] = {st[j].x, st[j].y, st[j].z, st[j].w};
          e4walk::store4_buf<S, 2>(e4walk::buffer_rsrc(head, bytes),
                                   static_cast<int>((static_cast<int64_t>(m) * a.stride_state_dim + n) * sizeof(SS)), w);
        } else {
          store4<S>(hstate + row_slot * a.stride_state_slot + n, st[j]);
        }
      }
      const f32x4 sc = st[j] * Cv[j];
      part += (sc.x + sc.y) + (sc.z + sc.w);
    }
#pragma unroll
    for (int w = LPR / 2; w > 0; w >>= 1) part += __shfl_xor(part, w);
    if (lr == 0 && mok)
      e4::store_scalar(a.out, tok * a.stride_out_tok + h * a.stride_out_head + m, a.out_dtype, part + x * Dh);

    // the state the next row starts from
    if (next >= 0) {
      if (dfs) {
        if ((pl & kPlanMulti) != 0) {  // several children: park the state, as a reload would give it, for the later ones
          if (sp < kStack) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              f32x4 w = st[j];
              if constexpr (!kExact)
                w = f32x4{e4::round_through<S>(w.x), e4::round_through<S>(w.y), e4::round_through<S>(w.z),
                          e4::round_through<S>(w.w)};
              my_stack[sp][j][lane] = w;
            }
            ++sp;
          } else {
            unparked |= 1ull << u;
          }
        }
        if (next_first) {
          if constexpr (!kExact) {
            if (next != u + 1) {  // not the chain child: it starts from the stored (rounded) state
#pragma unroll
              for (int j = 0; j < 4; ++j)
                st[j] = f32x4{e4::round_through<S>(st[j].x), e4::round_through<S>(st[j].y),
                              e4::round_through<S>(st[j].z), e4::round_through<S>(st[j].w)};
            }
          }
        } else {
          const int p = readlane(par, next);
          if ((unparked >> p) & 1) {
            load_slot(static_cast<int64_t>(readlane64(static_cast<uint64_t>(my_slot), p)));
            settle_loads();
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) st[j] = my_stack[sp - 1][j][lane];
            if (next_last) --sp;
          }
        }
      } else {
        // the reference's rule (:56-61): a row whose parent is not the previous row reloads the parent's slot
        const int64_t p = uni64(e4::ld(a.parents, b, next));
        if (p != next - 1) {
          load_slot(uni64(e4::ld(a.slots, b, p)));
          settle_loads();
        }
      }
    }
    u = next;
  }
}

template <int LPR>
int launch_lpr(const eagle4_mamba2_args& a, hipStream_t s) {
  const dim3 grid((a.head_dim + NT / LPR - 1) / (NT / LPR), a.batch, a.heads);
  switch (a.state_dtype) {
    case EAGLE4_F32: mamba2_tree_kernel<LPR, e4::F32><<<grid, NT, 0, s>>>(a); break;
    case EAGLE4_BF16: mamba2_tree_kernel<LPR, e4::Bf16><<<grid, NT, 0, s>>>(a); break;
    case EAGLE4_F16: mamba2_tree_kernel<LPR, e4::F16><<<grid, NT, 0, s>>>(a); break;
    default: return EAGLE4_NOT_COVERED;
  }
  return E4_LAUNCH_STATUS();
}

}  // namespace

extern "C" int eagle4_mamba2_tree_state_update(const eagle4_mamba2_args* a, void* stream) {
  if (a->batch == 0 || a->heads == 0 || a->head_dim == 0) return EAGLE4_OK;
  const auto fdt = [](int d) { return d == EAGLE4_BF16 || d == EAGLE4_F16 || d == EAGLE4_F32; };
  const int esz = a->in_dtype == EAGLE4_F32 ? 4 : 2, ssz = a->state_dtype == EAGLE4_F32 ? 4 : 2;
  const auto al = [](const void* p, int n) { return reinterpret_cast<uintptr_t>(p) % n == 0; };
  if (a->batch < 0 || a->batch > 65535 || a->heads < 0 || a->heads > 65535 || a->groups <= 0 ||
      a->heads % a->groups || a->head_dim < 0 || a->A == nullptr || a->slots.ptr == nullptr ||
      a->parents.ptr == nullptr || a->query_start_loc.ptr == nullptr || !fdt(a->state_dtype) ||
      !fdt(a->in_dtype) || !fdt(a->dt_dtype) || !fdt(a->out_dtype) ||
      ((a->D != nullptr || a->dt_bias != nullptr) && !fdt(a->param_dtype)) ||
      // 4-element chunks: 16-byte (fp32) / 8-byte (16-bit) vector accesses of the state and of B / C
      !al(a->state, 4 * ssz) || a->stride_state_slot % 4 || a->stride_state_head % 4 || a->stride_state_dim % 4 ||
      !al(a->B, 4 * esz) || !al(a->C, 4 * esz) || a->stride_B_tok % 4 || a->stride_B_group % 4 ||
      a->stride_C_tok % 4 || a->stride_C_group % 4)
    return EAGLE4_NOT_COVERED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (a->dstate) {
    case 64: return launch_lpr<4>(*a, s);
    case 128: return launch_lpr<8>(*a, s);
    case 256: return launch_lpr<16>(*a, s);
    default: return EAGLE4_NOT_COVERED;
  }
}
