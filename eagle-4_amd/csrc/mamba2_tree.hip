// Mamba2 tree verify (kernels/mamba2_tree.py): the selective state update of every tree node, each continuing from
// its parent, on gfx950.
//
// One workgroup per (block of head dims, request, head). The (head_dim x dstate) state is spread over the workgroup:
// LPR = dstate / 16 lanes share a head-dim row m, each holding 16 fp32 state elements as four 4-element chunks
// c = lane_in_row + LPR j (so a row's lanes write one contiguous run per store), a wave holds 64 / LPR rows and the
// four waves 256 / LPR. Every node updates the state in registers (exp(A dt) decay, dt B x input), stores it to its
// slot and reduces C . state over the row's lanes (xor shuffles). A node whose parent is the previous row continues
// from the registers; any other reloads its parent's stored state (rounded through the pool dtype, as the reference
// reads it); each lane reads back only elements it wrote itself, so no barrier is needed (:56-61 of the reference's
// walk; it syncs because its load and store layouts differ across threads). The walk is store-bound: every node writes
// head_dim x dstate state elements.

#include "common.h"

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int NT = 256;

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

// softplus as the reference writes it (:38-39): log(exp(dt) + 1) up to 20, dt above
E4_DEV float softplus(float dt) { return dt <= 20.f ? logf(expf(dt) + 1.f) : dt; }

template <int LPR, typename S>
__global__ __launch_bounds__(NT) void mamba2_tree_kernel(const eagle4_mamba2_args a) {
  using SS = typename S::storage;
  constexpr int ROWS = NT / LPR;
  const int b = blockIdx.y, h = blockIdx.z;
  const int lane = threadIdx.x & 63, lr = lane % LPR;
  const int m = blockIdx.x * ROWS + (threadIdx.x >> 6) * (64 / LPR) + lane / LPR;
  const bool mok = m < a.head_dim;
  const int64_t bos = e4::ld(a.query_start_loc, b);
  const int64_t seq = e4::ld(a.query_start_loc, b + 1) - bos;
  if (seq <= 0) return;
  const int g = h / (a.heads / a.groups);
  const int64_t pad = a.pad_slot_id;

  SS* const hstate = static_cast<SS*>(a.state) + h * a.stride_state_head + static_cast<int64_t>(m) * a.stride_state_dim;
  f32x4 s[4];
  auto load_slot = [&](int64_t slot) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 4 * (lr + LPR * j);
      s[j] = (slot != pad && mok) ? load4<S>(hstate + slot * a.stride_state_slot + n) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  const int64_t init_row = a.num_accepted.ptr != nullptr ? (e4::ld(a.num_accepted, b) - 1 > 0 ? e4::ld(a.num_accepted, b) - 1 : 0) : 0;
  load_slot(e4::ld(a.slots, b, init_row));

  const float A = a.A[h];
  const float Dh = a.D != nullptr ? e4::load_scalar(a.D, h, a.param_dtype) : 0.f;
  const float dtb = a.dt_bias != nullptr ? e4::load_scalar(a.dt_bias, h, a.param_dtype) : 0.f;
  for (int64_t t = 0; t < seq; ++t) {
    const int64_t tok = bos + t;
    const int64_t parent = e4::ld(a.parents, b, t);
    if (t > 0 && parent != t - 1) load_slot(e4::ld(a.slots, b, parent));
    const float x = mok ? e4::load_scalar(a.x, tok * a.stride_x_tok + h * a.stride_x_head + m, a.in_dtype) : 0.f;
    float dt = e4::load_scalar(a.dt, tok * a.stride_dt_tok + h * a.stride_dt_head, a.dt_dtype) + dtb;
    if (a.dt_softplus) dt = softplus(dt);
    const float dA = exp2f(1.4426950408889634f * (A * dt));
    const int64_t bo = tok * a.stride_B_tok + g * a.stride_B_group, co = tok * a.stride_C_tok + g * a.stride_C_group;
    float part = 0.f;
    const int64_t row_slot = e4::ld(a.slots, b, t);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = 4 * (lr + LPR * j);
      f32x4 Bv, Cv;
      if (a.in_dtype == EAGLE4_F32) {
        Bv = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.B) + bo + n);
        Cv = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.C) + co + n);
      } else if (a.in_dtype == EAGLE4_BF16) {
        Bv = load4<e4::Bf16>(static_cast<const uint16_t*>(a.B) + bo + n);
        Cv = load4<e4::Bf16>(static_cast<const uint16_t*>(a.C) + co + n);
      } else {
        Bv = load4<e4::F16>(static_cast<const uint16_t*>(a.B) + bo + n);
        Cv = load4<e4::F16>(static_cast<const uint16_t*>(a.C) + co + n);
      }
      const f32x4 dB = Bv * dt;
      s[j] = s[j] * dA + dB * x;
      if (row_slot != pad && mok) store4<S>(hstate + row_slot * a.stride_state_slot + n, s[j]);
      const f32x4 sc = s[j] * Cv;
      part += (sc.x + sc.y) + (sc.z + sc.w);
    }
#pragma unroll
    for (int w = LPR / 2; w > 0; w >>= 1) part += __shfl_xor(part, w);
    if (lr == 0 && mok)
      e4::store_scalar(a.out, tok * a.stride_out_tok + h * a.stride_out_head + m, a.out_dtype, part + x * Dh);
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
