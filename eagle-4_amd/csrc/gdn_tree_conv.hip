// Width-4 tree causal conv1d of a GDN verify on gfx950 (kernels/gdn_tree_conv.py:402-497).
//
// HBM-bound: per request it streams the nodes' inputs once, writes the outputs (and the windows) once, and touches
// three history columns plus the rolled state. One thread owns VEC adjacent channels of one request: its history
// columns stay in registers, every node's window is gathered through the ancestor table (three re-reads of an
// earlier node's row, L1/L2 hits), and the state roll is written as the nodes go (all history reads happen first).
// With unit channel stride VEC = 8 and every x / out access is one 16-byte load or store per node.

#include "common.h"

namespace {

template <typename T, int VEC>
struct Vec {
  typename T::storage v[VEC];
};

template <typename T, int VEC>
E4_DEV void load_vec(Vec<T, VEC>& out, const typename T::storage* p, int64_t stride, bool contiguous, int n) {
  if constexpr (VEC == 8) {
    if (contiguous) {
      const uint4 raw = *reinterpret_cast<const uint4*>(p);
      const uint16_t* h = reinterpret_cast<const uint16_t*>(&raw);
#pragma unroll
      for (int i = 0; i < 8; ++i) out.v[i] = h[i];
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i) out.v[i] = i < n ? p[i * stride] : typename T::storage(0);
}

template <typename T, int VEC>
E4_DEV void store_vec(typename T::storage* p, int64_t stride, bool contiguous, const Vec<T, VEC>& in) {
  if constexpr (VEC == 8) {
    if (contiguous) {
      uint4 raw;
      uint16_t* h = reinterpret_cast<uint16_t*>(&raw);
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = in.v[i];
      *reinterpret_cast<uint4*>(p) = raw;
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < VEC; ++i) p[i * stride] = in.v[i];
}

// One product of the upstream conv: 16-bit operands, product rounded to the 16-bit dtype, returned as fp32
// (kernels/gdn_tree_conv.py:225-229, 429-430).
template <typename T>
E4_DEV float product(typename T::storage x, typename T::storage w) {
  return e4::round_through<T>(T::to_f32(x) * T::to_f32(w));
}

template <typename T, int VEC>
__global__ __launch_bounds__(256) void tree_conv_kernel(const eagle4_conv_args a) {
  using S = typename T::storage;
  const int seq = blockIdx.y;
  const int c0 = (blockIdx.x * blockDim.x + threadIdx.x) * VEC;
  if (c0 >= a.dim) return;
  // _conv_request (:43-56)
  const int64_t slot = e4::ld(a.conv_state_indices, seq);
  int64_t bos = 0, num_tokens = a.seqlen, history = 0;
  if (a.query_start_loc.ptr != nullptr) {
    bos = e4::ld(a.query_start_loc, seq);
    num_tokens = e4::ld(a.query_start_loc, seq + 1) - bos;
  }
  if (a.num_accepted.ptr != nullptr) history = e4::ld(a.num_accepted, seq) - 1;
  if (!(slot > a.pad_slot_id && num_tokens > 0)) return;
  const int nvec = (a.dim - c0) < VEC ? (a.dim - c0) : VEC;  // a ragged last vector runs the scalar path
  const bool xc = a.stride_x_dim == 1 && nvec == VEC && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                  ((a.stride_x_token | a.stride_x_seq) & 7) == 0 && (c0 & 7) == 0;
  const bool oc = a.stride_o_dim == 1 && nvec == VEC && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
                  ((a.stride_o_token | a.stride_o_seq) & 7) == 0 && (c0 & 7) == 0;

  const S* x = static_cast<const S*>(a.x) + (a.query_start_loc.ptr != nullptr ? 0 : seq * a.stride_x_seq) +
               bos * a.stride_x_token + c0 * a.stride_x_dim;
  S* out = static_cast<S*>(a.out) + (a.query_start_loc.ptr != nullptr ? 0 : seq * a.stride_o_seq) +
           bos * a.stride_o_token + c0 * a.stride_o_dim;
  S* state = static_cast<S*>(a.conv_state) + slot * a.stride_cs_seq + c0 * a.stride_cs_dim;
  const S* w = static_cast<const S*>(a.weight) + c0 * a.stride_w_dim;

  float wt[4][VEC], bias[VEC];
  S col[3][VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const bool ok = i < nvec;
#pragma unroll
    for (int j = 0; j < 4; ++j) wt[j][i] = ok ? T::to_f32(w[i * a.stride_w_dim + j * a.stride_w_width]) : 0.f;
    bias[i] = (ok && a.bias != nullptr) ? e4::load_scalar(a.bias, c0 + i, a.bias_dtype) : 0.f;
#pragma unroll
    for (int j = 0; j < 3; ++j) col[j][i] = ok ? state[i * a.stride_cs_dim + (history + j) * a.stride_cs_tok] : S(0);
  }
  // weights as 16-bit operands of the rounded products
  S wq[4][VEC];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int i = 0; i < VEC; ++i) wq[j][i] = T::from_f32(wt[j][i]);

  const int32_t* anc = a.ancestors + static_cast<int64_t>(seq) * 3 * a.seqlen;
  const int64_t shift = (num_tokens + 2 < a.state_len ? num_tokens + 2 : a.state_len) - num_tokens - 3;
  S* window = nullptr;
  if (a.window != nullptr)
    window = static_cast<S*>(a.window) + e4::ld(a.window_indices, seq) * a.stride_win_seq + c0 * a.stride_win_dim;

  for (int64_t t = 0; t < num_tokens; ++t) {
    Vec<T, VEC> xs, v[3];
    load_vec<T, VEC>(xs, x + t * a.stride_x_token, a.stride_x_dim, xc, nvec);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int code = anc[j * a.seqlen + t];
      if (code >= 0) {
        load_vec<T, VEC>(v[j], x + static_cast<int64_t>(code) * a.stride_x_token, a.stride_x_dim, xc, nvec);
      } else {
        const int c = code == -1 ? 2 : (code == -2 ? 1 : 0);  // _window_value (:95-98)
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[j].v[i] = col[c][i];
      }
    }
    Vec<T, VEC> o;
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      float acc = bias[i];
      acc += product<T>(xs.v[i], wq[3][i]);  // self * w3, parent * w2, grandparent * w1, great-grandparent * w0
      acc += product<T>(v[0].v[i], wq[2][i]);
      acc += product<T>(v[1].v[i], wq[1][i]);
      acc += product<T>(v[2].v[i], wq[0][i]);
      if (a.silu) acc = acc / (1.0f + expf(-acc));
      o.v[i] = T::from_f32(acc);
    }
    if (nvec == VEC) {
      store_vec<T, VEC>(out + t * a.stride_o_token, a.stride_o_dim, oc, o);
    } else {
      for (int i = 0; i < nvec; ++i) out[t * a.stride_o_token + i * a.stride_o_dim] = o.v[i];
    }
    if (window != nullptr) {  // slot 0 grandparent, 1 parent, 2 self (:241-264)
      S* wp = window + t * a.stride_win_step;
      for (int i = 0; i < nvec; ++i) {
        wp[i * a.stride_win_dim + 0 * a.stride_win_win] = v[1].v[i];
        wp[i * a.stride_win_dim + 1 * a.stride_win_win] = v[0].v[i];
        wp[i * a.stride_win_dim + 2 * a.stride_win_win] = xs.v[i];
      }
    }
    // the roll (:266-278): input t goes to column t + 3 + shift; every history read is already done
    const int64_t dest = t + 3 + shift;
    if (dest >= 0)
      for (int i = 0; i < nvec; ++i) state[i * a.stride_cs_dim + dest * a.stride_cs_tok] = xs.v[i];
  }
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int64_t dest = j + shift;
    if (dest >= 0)
      for (int i = 0; i < nvec; ++i) state[i * a.stride_cs_dim + dest * a.stride_cs_tok] = col[j][i];
  }
}

}  // namespace

extern "C" int eagle4_gdn_tree_conv1d_update(const eagle4_conv_args* a, void* stream) {
  if (a->batch == 0 || a->dim == 0) return EAGLE4_OK;
  if ((a->dtype != EAGLE4_BF16 && a->dtype != EAGLE4_F16) || a->state_len < 3 || a->seqlen < 1 ||
      a->conv_state_indices.ptr == nullptr || a->ancestors == nullptr ||
      (a->window != nullptr && a->window_indices.ptr == nullptr))
    return EAGLE4_NOT_COVERED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr int kVec = 8;
  const dim3 grid(e4::ceil_div(e4::ceil_div(a->dim, kVec), 256), a->batch);
  if (a->dtype == EAGLE4_BF16)
    tree_conv_kernel<e4::Bf16, kVec><<<grid, 256, 0, s>>>(*a);
  else
    tree_conv_kernel<e4::F16, kVec><<<grid, 256, 0, s>>>(*a);
  return E4_LAUNCH_STATUS();
}
