// Width-4 tree causal conv1d of a GDN verify on gfx950 (kernels/gdn_tree_conv.py:402-497).
//
// Per request it reads the nodes' inputs, the history columns of the conv state and the weights once, and writes the
// outputs, the windows and the rolled state once. One workgroup takes one request and a block of kChannels channels
// (a thread per channel for the roll, an 8-channel octet per thread and node for the outputs). It stages the block's
// node inputs (token-major, 16 bytes per 8 channels, LDS DMA when the rows are 16-byte vectors), the ancestor codes,
// the weights and the history in LDS; every thread then computes the outputs of its octet for a strided set of
// nodes, each window gathered from LDS through the ancestor table, and the roll follows. The kernel is a chain of
// latencies (lookups, staging, outputs, roll) per workgroup, so it is sized for residency: at most 64 VGPRs and
// ~20 KB of LDS at 16 nodes and 19-column rows, eight workgroups per CU, so a batch-64 launch of 2048 workgroups is
// resident at once.
//
// When the state rows are contiguous (token stride 1, channel stride = state length: the block's rows are one
// 16-byte-aligned span of kChannels * L elements) the span is copied into LDS by direct loads, each thread reads its
// channel's history columns and later writes its channel's rolled row back into the copy (the loop over columns is
// the same for every thread: no divergence), and the span leaves with 16-byte stores, so no cache line is left partly
// written and the span is read once. Otherwise the history is read element by element and the roll written element
// by element along the contiguous dimension.

#include "common.h"

namespace {

constexpr int kChannels = 256;          // channels per workgroup
constexpr int kVecs = kChannels / 8;    // 8-channel vectors per node
constexpr int kThreads = 256;
constexpr int kTokLanes = kThreads / kVecs;  // nodes computed concurrently
constexpr int kMaxNodes = 64;
constexpr int kTokPerDma = 64 / kVecs;  // node inputs per 1 KB direct load
static_assert(kVecs <= 64 && 64 % kVecs == 0, "a direct load covers whole node inputs");
static_assert(kThreads == kChannels, "a thread per channel for the roll");
constexpr int kMaxSpan = 24 * 1024;    // bytes of a block's state rows staged for the roll (rows up to 48 columns),
                                        // so the LDS stays within the 64 KB a launch gets without attributes

// Two products of the upstream conv: 16-bit operands, each product rounded to nearest even in the 16-bit dtype and
// returned as fp32 (kernels/gdn_tree_conv.py:225-229, 429-430); for bf16 one v_cvt_pk_bf16_f32 rounds both.
typedef float f32x2 __attribute__((ext_vector_type(2)));
template <typename T>
E4_DEV f32x2 product2(uint16_t x0, uint16_t x1, float w0, float w1) {
  const f32x2 p = {T::to_f32(x0) * w0, T::to_f32(x1) * w1};
  if constexpr (T::code == EAGLE4_BF16) {
    uint32_t r;  // both rounded by one instruction (the compiler splits a vector conversion here)
    asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(r) : "v"(p.x), "v"(p.y));
    return f32x2{__uint_as_float(r << 16), __uint_as_float(r & 0xffff0000u)};
  } else {
    return f32x2{static_cast<float>(static_cast<_Float16>(p.x)), static_cast<float>(static_cast<_Float16>(p.y))};
  }
}

// x sigmoid(x) = x / (1 + e^-x), e^-x as 2^(-x log2 e) on v_exp_f32 and the quotient on v_rcp_f32.
E4_DEV float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

E4_DEV uint16_t lane16(const uint4& v, int i) {
  const uint32_t w = i < 4 ? (i < 2 ? v.x : v.y) : (i < 6 ? v.z : v.w);
  return static_cast<uint16_t>((i & 1) ? (w >> 16) : (w & 0xffffu));
}

// 64 lanes x 16 bytes from per-lane global addresses into LDS [dst, dst + 1024), lane p at dst + 16 p.
// (nontemporal policy: the inputs and state rows are read once; batch-64 step 0.771 -> 0.764 ms)
E4_DEV void dma16(const void* src, char* dst) { __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 2); }

// LDS layout (byte offsets): node inputs [seqlen rounded up to kTokPerDma][kVecs] x 16, the state span [kChannels][L]
// x 2 (row roll; the history columns are read from it) or history [3][kChannels] x 2 (element-wise state), weights
// [4][kChannels] x 2 (the raw 16-bit taps), ancestor codes [3][seqlen].
struct Lds {
  int xs, rows, hist, wts, anc, total;
  int row_roll;  // the state span is staged in LDS and written back whole
};

Lds lds_layout(const eagle4_conv_args& a) {
  auto up16 = [](int b) { return (b + 15) / 16 * 16; };
  Lds l;
  l.row_roll = a.stride_cs_tok == 1 && a.stride_cs_dim == a.state_len && kChannels * a.state_len * 2 <= kMaxSpan &&
               a.dim % kChannels == 0 && (reinterpret_cast<uintptr_t>(a.conv_state) & 15) == 0 &&
               (a.stride_cs_seq * 2) % 16 == 0;
  l.xs = 0;
  l.rows = (a.seqlen + kTokPerDma - 1) / kTokPerDma * 1024;
  l.hist = l.rows + (l.row_roll ? up16(kChannels * a.state_len * 2) : 0);
  l.wts = l.hist + (l.row_roll ? 0 : up16(3 * kChannels * 2));
  l.anc = l.wts + 4 * kChannels * 2;
  l.total = l.anc + up16(3 * a.seqlen * 4);
  return l;
}

// kFast: the common layout — contiguous 16-byte-aligned node inputs, outputs and state rows (row roll), no windows —
// with the other paths compiled out, so the kernel fits in 64 VGPRs (eight workgroups per CU).
template <typename T, bool kFast>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(kFast ? 8 : 5)))
void tree_conv_kernel(const eagle4_conv_args a, const Lds off) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint4* const xs = reinterpret_cast<uint4*>(lds + off.xs);        // [t * kVecs + v]
  uint16_t* const rows = reinterpret_cast<uint16_t*>(lds + off.rows);  // [c * L + col] (row roll)
  uint16_t* const hist = reinterpret_cast<uint16_t*>(lds + off.hist);  // [j * kChannels + c] (element-wise state)
  uint16_t* const wts = reinterpret_cast<uint16_t*>(lds + off.wts);    // [j * kChannels + c]
  int* const anc = reinterpret_cast<int*>(lds + off.anc);             // [j * n + t]
  const int seq = blockIdx.y;
  const int cb = blockIdx.x * kChannels;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int L = a.state_len;

  // _conv_request (:43-56)
  const int64_t slot = e4::ld(a.conv_state_indices, seq);
  int64_t bos = 0, num_tokens = a.seqlen, history = 0;
  if (a.query_start_loc.ptr != nullptr) {
    bos = e4::ld(a.query_start_loc, seq);
    num_tokens = e4::ld(a.query_start_loc, seq + 1) - bos;
  }
  if (a.num_accepted.ptr != nullptr) history = e4::ld(a.num_accepted, seq) - 1;
  if (!(slot > a.pad_slot_id && num_tokens > 0)) return;
  const int n = static_cast<int>(num_tokens < a.seqlen ? num_tokens : a.seqlen);
  const int nch = a.dim - cb < kChannels ? a.dim - cb : kChannels;

  const uint16_t* x = static_cast<const uint16_t*>(a.x) +
                      (a.query_start_loc.ptr != nullptr ? 0 : seq * a.stride_x_seq) + bos * a.stride_x_token +
                      static_cast<int64_t>(cb) * a.stride_x_dim;
  uint16_t* out = static_cast<uint16_t*>(a.out) + (a.query_start_loc.ptr != nullptr ? 0 : seq * a.stride_o_seq) +
                  bos * a.stride_o_token + static_cast<int64_t>(cb) * a.stride_o_dim;
  uint16_t* state = static_cast<uint16_t*>(a.conv_state) + slot * a.stride_cs_seq +
                    static_cast<int64_t>(cb) * a.stride_cs_dim;

  // ---- stage: the state span, node inputs, ancestor codes, weights, bias ------------------------------------------
  const int span = kChannels * L / 8;  // 16-byte pieces of the block's state rows (row roll)
  const bool row_roll = kFast || off.row_roll;
  if (row_roll) {  // instruction k fills pieces 64 k .. 64 k + 63 (lanes past the span are off)
    for (int k = wave; 64 * k < span; k += kThreads / 64) {
      if (64 * k + lane < span) dma16(reinterpret_cast<const char*>(state) + 16 * (64 * k + lane), lds + off.rows + k * 1024);
    }
  }
  const bool xvec = kFast || (a.stride_x_dim == 1 && nch == kChannels && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 &&
                              ((a.stride_x_token | a.stride_x_seq | cb) & 7) == 0);
  if (xvec) {  // instruction m fills tokens kTokPerDma m .. + kTokPerDma - 1 (past the last token: the last again)
    for (int m = wave; kTokPerDma * m < n; m += kThreads / 64) {
      const int t0 = kTokPerDma * m + lane / kVecs, t = t0 < n ? t0 : n - 1;
      dma16(x + t * a.stride_x_token + 8 * (lane % kVecs), lds + off.xs + m * 1024);
    }
  } else {
    for (int i = tid; i < n * kVecs; i += kThreads) {
      const int t = i / kVecs, v = i % kVecs;
      const uint16_t* p = x + t * a.stride_x_token + 8 * v * a.stride_x_dim;
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = 8 * v + e < nch ? p[e * a.stride_x_dim] : 0u;
      xs[i] = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
    }
  }
  const int32_t* atab = a.ancestors + static_cast<int64_t>(seq) * 3 * a.seqlen;
  for (int i = tid; i < 3 * n; i += kThreads) anc[i] = atab[(i / n) * a.seqlen + i % n];
  {
    const bool tap_fast = a.stride_w_width == 1;  // lanes along the weight's contiguous dimension
    const uint16_t* wsrc = static_cast<const uint16_t*>(a.weight) + static_cast<int64_t>(cb) * a.stride_w_dim;
    for (int i = tid; i < 4 * kChannels; i += kThreads) {
      const int c = tap_fast ? i / 4 : i % kChannels, j = tap_fast ? i % 4 : i / kChannels;
      wts[j * kChannels + c] = c < nch ? wsrc[c * a.stride_w_dim + j * a.stride_w_width] : 0;
    }
  }
  const bool tok_fast = a.stride_cs_tok == 1;  // lanes along the state's contiguous dimension
  if (!row_roll) {
    for (int i = tid; i < 3 * kChannels; i += kThreads) {
      const int c = tok_fast ? i / 3 : i % kChannels, j = tok_fast ? i % 3 : i / kChannels;
      hist[j * kChannels + c] = c < nch ? state[c * a.stride_cs_dim + (history + j) * a.stride_cs_tok] : 0;
    }
  }
  // this thread's octet of the bias, as raw bits, loaded with the staging so that the wait below covers it (a load
  // left in flight here would make the compiler wait for every store before the roll)
  uint32_t bias_raw[8];
  {
    const int c0 = 8 * (tid % kVecs);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bias_raw[e] = 0u;
      if (a.bias != nullptr && c0 + e < nch) {
        const int64_t i = cb + c0 + e;
        bias_raw[e] = a.bias_dtype == EAGLE4_F32 ? static_cast<const uint32_t*>(a.bias)[i]
                                                 : static_cast<const uint16_t*>(a.bias)[i];
      }
    }
  }
  // the direct loads have landed: vmcnt(0) as the builtin, which the compiler's own wait placement sees (after an
  // opaque asm wait it would wait again before the first LDS read behind every direct load, and that wait would
  // also cover the output stores issued by then: the roll behind all of them)
  if (xvec || row_roll) __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();

  // ---- outputs: thread (token lane tl, vector v) computes channels 8 v .. 8 v + 7 of nodes tl, tl + kTokLanes, ... ---
  {
    const int v = tid % kVecs, tl = tid / kVecs;
    const int c0 = 8 * v;
    const bool ovec = kFast || (a.stride_o_dim == 1 && nch == kChannels && (reinterpret_cast<uintptr_t>(a.out) & 15) == 0 &&
                                ((a.stride_o_token | a.stride_o_seq | cb) & 7) == 0);
    uint16_t* window = nullptr;
    if (!kFast && a.window != nullptr)
      window = static_cast<uint16_t*>(a.window) + e4::ld(a.window_indices, seq) * a.stride_win_seq +
               static_cast<int64_t>(cb + c0) * a.stride_win_dim;
    float bias[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      bias[e] = a.bias_dtype == EAGLE4_F32    ? __uint_as_float(bias_raw[e])
                : a.bias_dtype == EAGLE4_BF16 ? e4::bf16_to_f32(static_cast<uint16_t>(bias_raw[e]))
                                              : e4::f16_to_f32(static_cast<uint16_t>(bias_raw[e]));
    for (int t = tl; t < n; t += kTokLanes) {
      const uint4 xt = xs[t * kVecs + v];
      uint4 win[3];  // parent, grandparent, great-grandparent
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int code = anc[j * n + t];
        // _window_value (:95-98): history column 2 (code -1), 1 (-2), 0 (-3)
        if (code >= 0) {
          win[j] = xs[code * kVecs + v];
        } else if (row_roll) {  // the octet's history column out of the staged rows
          const uint16_t* hp = rows + c0 * L + history + (code + 3);
          uint32_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = hp[e * L];
          win[j] = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
        } else {
          win[j] = *reinterpret_cast<const uint4*>(&hist[(code + 3) * kChannels + c0]);
        }
      }
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        // channels e, e + 1 together; per channel the sum in the reference's order: bias, then self w3, parent w2,
        // grandparent w1, great-grandparent w0; the taps of the pair, one 32-bit read per tap
        float wv[4][2];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t wp = *reinterpret_cast<const uint32_t*>(&wts[j * kChannels + c0 + e]);
          wv[j][0] = T::to_f32(static_cast<uint16_t>(wp & 0xffffu));
          wv[j][1] = T::to_f32(static_cast<uint16_t>(wp >> 16));
        }
        const f32x2 p3 = product2<T>(lane16(xt, e), lane16(xt, e + 1), wv[3][0], wv[3][1]);
        const f32x2 p2 = product2<T>(lane16(win[0], e), lane16(win[0], e + 1), wv[2][0], wv[2][1]);
        const f32x2 p1 = product2<T>(lane16(win[1], e), lane16(win[1], e + 1), wv[1][0], wv[1][1]);
        const f32x2 p0 = product2<T>(lane16(win[2], e), lane16(win[2], e + 1), wv[0][0], wv[0][1]);
        float r[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          float acc = bias[e + k];
          acc += p3[k];
          acc += p2[k];
          acc += p1[k];
          acc += p0[k];
          if (a.silu) acc = silu(acc);
          r[k] = acc;
        }
        if constexpr (T::code == EAGLE4_BF16) {  // both rounded to nearest even by one instruction
          asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(o[e / 2]) : "v"(r[0]), "v"(r[1]));
        } else {
          o[e / 2] = static_cast<uint32_t>(T::from_f32(r[0])) | static_cast<uint32_t>(T::from_f32(r[1])) << 16;
        }
      }
      uint16_t* op = out + t * a.stride_o_token + c0 * a.stride_o_dim;
      if (ovec) {
        typedef uint32_t u32x4o __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(u32x4o{o[0], o[1], o[2], o[3]}, reinterpret_cast<u32x4o*>(op));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (c0 + e < nch) op[e * a.stride_o_dim] = static_cast<uint16_t>((e & 1) ? o[e / 2] >> 16 : o[e / 2] & 0xffffu);
      }
      if (window != nullptr) {  // slot 0 grandparent, 1 parent, 2 self (:241-264)
        uint16_t* wp = window + t * a.stride_win_step;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (c0 + e >= nch) break;
          wp[e * a.stride_win_dim + 0 * a.stride_win_win] = lane16(win[1], e);
          wp[e * a.stride_win_dim + 1 * a.stride_win_win] = lane16(win[0], e);
          wp[e * a.stride_win_dim + 2 * a.stride_win_win] = lane16(xt, e);
        }
      }
    }
  }

  // ---- the roll (:266-278): history column j goes to column j + shift, node t's input to t + 3 + shift (kept when
  // the column is >= 0); every history read was staged before the barrier --------------------------------------------
  const int shift = static_cast<int>((num_tokens + 2 < L ? num_tokens + 2 : L) - num_tokens - 3);
  const int cols = 3 + n;  // source columns: history 0..2, then the nodes
  if (row_roll) {
    // this thread's channel: the destination columns in order (the same loop in every thread), into the staged span,
    // once every output's history reads of the span are done; the channel's history columns are read first
    __syncthreads();
    const int c = tid;
    const uint16_t h0 = rows[c * L + history], h1 = rows[c * L + history + 1], h2 = rows[c * L + history + 2];
    const int lo = shift > 0 ? shift : 0, hi = cols + shift < L ? cols + shift : L;
    for (int col = lo; col < hi; ++col) {
      const int src = col - shift;
      rows[c * L + col] = src == 0 ? h0 : src == 1 ? h1 : src == 2 ? h2 : lane16(xs[(src - 3) * kVecs + c / 8], c % 8);
    }
    __syncthreads();
    const uint4* staged = reinterpret_cast<const uint4*>(rows);
    uint4* dst = reinterpret_cast<uint4*>(state);
    // nontemporal: the rolled rows are read again only by the next round's conv (batch-64 step 0.740 -> 0.736 ms)
    typedef uint32_t u32x4n __attribute__((ext_vector_type(4)));
    for (int i = tid; i < span; i += kThreads) {
      const uint4 w = staged[i];
      __builtin_nontemporal_store(u32x4n{w.x, w.y, w.z, w.w}, reinterpret_cast<u32x4n*>(dst + i));
    }
  } else {
    for (int i = tid; i < cols * kChannels; i += kThreads) {
      const int c = tok_fast ? i / cols : i % kChannels, src = tok_fast ? i % cols : i / kChannels;
      const int64_t dest = src + shift;
      if (c >= nch || dest < 0) continue;
      const uint16_t val = src < 3 ? hist[src * kChannels + c] : lane16(xs[(src - 3) * kVecs + c / 8], c % 8);
      state[c * a.stride_cs_dim + dest * a.stride_cs_tok] = val;
    }
  }
}

}  // namespace

extern "C" int eagle4_gdn_tree_conv1d_update(const eagle4_conv_args* a, void* stream) {
  if (a->batch == 0 || a->dim == 0) return EAGLE4_OK;
  if ((a->dtype != EAGLE4_BF16 && a->dtype != EAGLE4_F16) || a->state_len < 3 || a->seqlen < 1 ||
      a->seqlen > kMaxNodes || a->conv_state_indices.ptr == nullptr || a->ancestors == nullptr ||
      (a->window != nullptr && a->window_indices.ptr == nullptr))
    return EAGLE4_NOT_COVERED;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const Lds off = lds_layout(*a);
  const dim3 grid(e4::ceil_div(a->dim, kChannels), a->batch);
  // the kernel's vector conditions, for every block (dim a multiple of kChannels) and request
  auto vec = [&](const void* p, int64_t s_dim, int64_t s_tok, int64_t s_seq) {
    return s_dim == 1 && a->dim % kChannels == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0 && ((s_tok | s_seq) & 7) == 0;
  };
  const bool fast = off.row_roll && a->window == nullptr && vec(a->x, a->stride_x_dim, a->stride_x_token, a->stride_x_seq) &&
                    vec(a->out, a->stride_o_dim, a->stride_o_token, a->stride_o_seq);
  if (a->dtype == EAGLE4_BF16) {
    if (fast)
      tree_conv_kernel<e4::Bf16, true><<<grid, kThreads, off.total, s>>>(*a, off);
    else
      tree_conv_kernel<e4::Bf16, false><<<grid, kThreads, off.total, s>>>(*a, off);
  } else {
    if (fast)
      tree_conv_kernel<e4::F16, true><<<grid, kThreads, off.total, s>>>(*a, off);
    else
      tree_conv_kernel<e4::F16, false><<<grid, kThreads, off.total, s>>>(*a, off);
  }
  return E4_LAUNCH_STATUS();
}
