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

// Four raw input values (q or k) as loaded: a float4 for fp32 inputs, four 16-bit values in a uint2 otherwise.
template <typename T>
using Raw4 = typename std::conditional<sizeof(typename T::storage) == 4, float4, uint2>::type;

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
