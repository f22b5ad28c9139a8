// Device helpers shared by the GDN tree walks (gdn_tree_recurrence.hip: snapshot contract; gdn_tree_records.hip:
// records contract): state chunk loads and stores, raw input loads widened where they are used, the gate, lane
// broadcasts, and the per-node inputs a lane holds.
#pragma once

#include <type_traits>

#include "common.h"

namespace e4walk {

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

// Stores go through native vector types: HIP's float4 / uint2 structs compile the walk's snapshot stores with extra
// register moves (453 against 448 us for the batch-64 walk).
template <typename T>
E4_DEV void store4(typename T::storage* p, const float* in) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(typename T::storage) == 4) {
    *reinterpret_cast<f32x4v*>(p) = f32x4v{in[0], in[1], in[2], in[3]};
  } else {
    u32x2v v;
    v.x = static_cast<uint32_t>(T::from_f32(in[0])) | (static_cast<uint32_t>(T::from_f32(in[1])) << 16);
    v.y = static_cast<uint32_t>(T::from_f32(in[2])) | (static_cast<uint32_t>(T::from_f32(in[3])) << 16);
    *reinterpret_cast<u32x2v*>(p) = v;
  }
}

// The same through a buffer resource, with cache policy AUX (2: nontemporal, which leaves no dirty line in the
// last-level cache for the next kernel to write back). The policy is an immediate operand, so the compiler cannot
// merge this store with a regular one on another path and drop the policy, as it does with nontemporal metadata.
template <typename T, int AUX>
E4_DEV void store4_buf(__amdgpu_buffer_rsrc_t r, int byte_off, const float* in) {
  typedef unsigned u32x4v __attribute__((ext_vector_type(4)));
  typedef unsigned u32x2v __attribute__((ext_vector_type(2)));
  if constexpr (sizeof(typename T::storage) == 4) {
    const u32x4v v = {__float_as_uint(in[0]), __float_as_uint(in[1]), __float_as_uint(in[2]), __float_as_uint(in[3])};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, AUX);
  } else {
    const u32x2v v = {static_cast<uint32_t>(T::from_f32(in[0])) | (static_cast<uint32_t>(T::from_f32(in[1])) << 16),
                      static_cast<uint32_t>(T::from_f32(in[2])) | (static_cast<uint32_t>(T::from_f32(in[3])) << 16)};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, byte_off, 0, AUX);
  }
}

// A buffer resource over [base, base + bytes) (raw: byte offsets, 32-bit data format).
E4_DEV __amdgpu_buffer_rsrc_t buffer_rsrc(void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
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

// Native vectors: arrays of them stay in registers (arrays of HIP's float4 / uint4 structs can land in scratch memory).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Four raw input values (q or k) as loaded: 16 bytes of fp32, or four 16-bit values in 8 bytes.
template <typename T>
using Raw4 = typename std::conditional<sizeof(typename T::storage) == 4, f32x4, u32x2>::type;

template <typename T>
E4_DEV void widen4(const Raw4<T>& r, float* out) {
  if constexpr (sizeof(typename T::storage) == 4) {
    out[0] = r.x;
    out[1] = r.y;
    out[2] = r.z;
    out[3] = r.w;
  } else {
    out[0] = T::to_f32(static_cast<uint16_t>(r.x & 0xffffu));
    out[1] = T::to_f32(static_cast<uint16_t>(r.x >> 16));
    out[2] = T::to_f32(static_cast<uint16_t>(r.y & 0xffffu));
    out[3] = T::to_f32(static_cast<uint16_t>(r.y >> 16));
  }
}

// A gate value of a runtime dtype, as raw bits (loaded here, widened where it is used: a conversion next to its load
// would make the compiler wait for every store in flight too, since vmcnt counts stores).
E4_DEV uint32_t load_raw(const void* p, int64_t i, int dtype) {
  if (dtype == EAGLE4_F32) return static_cast<const uint32_t*>(p)[i];
  return static_cast<const uint16_t*>(p)[i];
}

E4_DEV float widen_raw(uint32_t r, int dtype) {
  if (dtype == EAGLE4_F32) return __uint_as_float(r);
  if (dtype == EAGLE4_BF16) return e4::bf16_to_f32(static_cast<uint16_t>(r));
  return e4::f16_to_f32(static_cast<uint16_t>(r));
}

// The gate of a node (kernels/gdn_tree_recurrence.py:115-140): the decay exp(g), g = -exp(A_log) softplus(a + dt_bias)
// (linear above the threshold), and the write strength beta = sigmoid(b) rounded through b's dtype. A = -exp(A_log).
E4_DEV float2 gate_of(uint32_t a_raw, uint32_t b_raw, int gate_dtype, float softplus_beta, float softplus_threshold,
                      float A, float dt_bias) {
  const float x = widen_raw(a_raw, gate_dtype) + dt_bias;
  const float bx = softplus_beta * x;
  const float softplus = bx <= softplus_threshold ? (1.0f / softplus_beta) * logf(1.0f + expf(bx)) : x;
  const float decay = expf(A * softplus);
  const float beta = e4::round_code(1.0f / (1.0f + expf(-widen_raw(b_raw, gate_dtype))), gate_dtype);
  return make_float2(decay, beta);
}

// Waits for every vector memory operation of the wave (vmcnt(0); expcnt and lgkmcnt untouched). Placed right after a
// load on a rarely taken path, it settles the loaded registers there, so the compiler does not wait for them (and with
// them for every store in flight) where that path joins the main one.
E4_DEV void settle_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

E4_DEV int readlane(int x, int l) { return __builtin_amdgcn_readlane(x, l); }

// A value every lane holds the same copy of (a request's table entries), moved to a scalar register so the code
// that depends on it (the walk's loop bounds and branches) is compiled as wave-uniform, not per lane.
E4_DEV int uni(int x) { return __builtin_amdgcn_readfirstlane(x); }
E4_DEV int64_t uni64(int64_t x) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint64_t>(x) & 0xffffffffu));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint64_t>(x) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}
E4_DEV uint64_t readlane64(uint64_t x, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(x & 0xffffffffu), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(x >> 32), l);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// One node's inputs in a lane's registers: its E values of q and k (raw), v of its RPT rows (raw), and the node's
// scalars (decay, beta, qs = scale / |q|, ks = 1 / |k|).
template <int E, int RPT, typename Tin>
struct Node {
  Raw4<Tin> q[E / 4], k[E / 4];
  typename Tin::storage v[RPT];
  float4 sc;
};

}  // namespace e4walk

namespace e4walk {

// ---- a walk's prologue: every load issued before the first wait -------------------------------------------------
// Four state values of a runtime dtype as raw bits (16 bytes of fp32, or 8 bytes of a 16-bit dtype in .x / .y),
// widened later: a conversion next to each load would make every load wait for the one before.
E4_DEV void load_state_raw(const void* base, int64_t off, int dtype, u32x4& r) {
  if (dtype == EAGLE4_F32) {
    r = *reinterpret_cast<const u32x4*>(static_cast<const float*>(base) + off);
  } else {
    const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
    r = u32x4{t.x, t.y, 0u, 0u};
  }
}

E4_DEV void widen_state_raw(const u32x4& r, int dtype, float* out) {
  if (dtype == EAGLE4_F32) {
    out[0] = __uint_as_float(r.x);
    out[1] = __uint_as_float(r.y);
    out[2] = __uint_as_float(r.z);
    out[3] = __uint_as_float(r.w);
  } else {
    const uint16_t v[4] = {static_cast<uint16_t>(r.x & 0xffffu), static_cast<uint16_t>(r.x >> 16),
                           static_cast<uint16_t>(r.y & 0xffffu), static_cast<uint16_t>(r.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = dtype == EAGLE4_BF16 ? e4::bf16_to_f32(v[e]) : e4::f16_to_f32(v[e]);
  }
}

// Where a request's node inputs live: q, k rows of its key head, v rows of its value head, gate inputs.
struct NodeSrc {
  const void *q, *k, *v, *a, *b;
  int64_t stride_q, stride_k, stride_v, stride_a, stride_b;
  int gate_dtype, ih, hv, V;
};

// The inputs of nodes [0, ts) of a request (ts <= TS), loaded by NT threads into registers (issue) and then written
// to LDS (commit), so all their loads are in flight together. The workgroup's V rows are [row0, row0 + ROWS).
template <typename Tin, int K, int TS, int ROWS, int NT>
struct Staging {
  using IS = typename Tin::storage;
  static constexpr int CH = K / 4;  // Raw4 chunks per q / k row
  static constexpr int QK_IT = (TS * CH + NT - 1) / NT;
  static constexpr int V_IT = (TS * ROWS + NT - 1) / NT;
  Raw4<Tin> q[QK_IT], k[QK_IT];
  IS v[V_IT];
  uint32_t ga, gb;

  E4_DEV void issue(const NodeSrc& s, int64_t bos, int ts, int row0, int tid) {
#pragma unroll
    for (int it = 0; it < QK_IT; ++it) {
      const int i = tid + it * NT;
      if (i < ts * CH) {
        const int t = i / CH, ch = i % CH;
        const int64_t tok = bos + t;
        q[it] = *reinterpret_cast<const Raw4<Tin>*>(static_cast<const IS*>(s.q) + tok * s.stride_q +
                                                    static_cast<int64_t>(s.ih) * K + 4 * ch);
        k[it] = *reinterpret_cast<const Raw4<Tin>*>(static_cast<const IS*>(s.k) + tok * s.stride_k +
                                                    static_cast<int64_t>(s.ih) * K + 4 * ch);
      }
    }
#pragma unroll
    for (int it = 0; it < V_IT; ++it) {
      const int i = tid + it * NT;
      if (i < ts * ROWS) {
        const int t = i / ROWS, r = i % ROWS;
        const int row = row0 + r < s.V ? row0 + r : s.V - 1;  // rows past V are computed and dropped
        v[it] = static_cast<const IS*>(s.v)[(bos + t) * s.stride_v + static_cast<int64_t>(s.hv) * s.V + row];
      }
    }
    if (tid < ts) {
      ga = load_raw(s.a, (bos + tid) * s.stride_a + s.hv, s.gate_dtype);
      gb = load_raw(s.b, (bos + tid) * s.stride_b + s.hv, s.gate_dtype);
    }
  }

  E4_DEV void commit(IS (&s_q)[TS][K], IS (&s_k)[TS][K], IS (&s_v)[TS][ROWS], float4 (&s_sc)[TS], int ts, int tid,
                     int gate_dtype, float softplus_beta, float softplus_threshold, float A, float dt_bias) {
#pragma unroll
    for (int it = 0; it < QK_IT; ++it) {
      const int i = tid + it * NT;
      if (i < ts * CH) {
        const int t = i / CH, ch = i % CH;
        *reinterpret_cast<Raw4<Tin>*>(&s_q[t][4 * ch]) = q[it];
        *reinterpret_cast<Raw4<Tin>*>(&s_k[t][4 * ch]) = k[it];
      }
    }
#pragma unroll
    for (int it = 0; it < V_IT; ++it) {
      const int i = tid + it * NT;
      if (i < ts * ROWS) s_v[i / ROWS][i % ROWS] = v[it];
    }
    if (tid < ts) {
      const float2 g = gate_of(ga, gb, gate_dtype, softplus_beta, softplus_threshold, A, dt_bias);
      s_sc[tid] = make_float4(g.x, g.y, 0.f, 0.f);
    }
  }
};

// L2 norms over K of the staged nodes (kernels/gdn_tree_recurrence.py:143-151), all nodes at once: NT / TS
// adjacent threads share a node, each summing a contiguous run of its q and k; .z = scale / |q|, .w = 1 / |k|
// (1e-6 inside the square roots). With qh / kh, every thread also writes its run of q^ = q .z and k^ = k .w there
// (the same products the separate pass makes), so no second pass over the raw rows follows.
template <typename Tin, int K, int TS, int NT>
E4_DEV void stage_norms(const typename Tin::storage (&s_q)[TS][K], const typename Tin::storage (&s_k)[TS][K],
                        float4 (&s_sc)[TS], int ts, int tid, float scale, float (*qh)[K] = nullptr,
                        float (*kh)[K] = nullptr) {
  constexpr int LPN0 = NT / TS < 64 ? NT / TS : 64;
  constexpr int LPN = LPN0 < K ? LPN0 : K;  // threads per node (a power of two)
  constexpr int PER = K / LPN;                       // elements each
  static_assert(PER >= 1 && K % LPN == 0, "norm split");
  const int t = tid / LPN, part = tid % LPN;
  float qq = 0.f, kk = 0.f;
  float qv[PER], kv[PER];
  if (t < ts) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      qv[e] = Tin::to_f32(s_q[t][part * PER + e]);
      kv[e] = Tin::to_f32(s_k[t][part * PER + e]);
      qq = fmaf(qv[e], qv[e], qq);
      kk = fmaf(kv[e], kv[e], kk);
    }
  }
  qq = e4::group_sum<LPN>(qq);
  kk = e4::group_sum<LPN>(kk);
  const float qs = scale / sqrtf(qq + 1e-6f), ks = 1.0f / sqrtf(kk + 1e-6f);
  if (t < ts && part == 0) {
    s_sc[t].z = qs;
    s_sc[t].w = ks;
  }
  if (qh != nullptr && t < ts) {
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      qh[t][part * PER + e] = qv[e] * qs;
      kh[t][part * PER + e] = kv[e] * ks;
    }
  }
}

}  // namespace e4walk
