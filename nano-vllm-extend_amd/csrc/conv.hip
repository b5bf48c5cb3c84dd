// Depthwise causal conv1d (width K = 4) + SiLU over the packed qkv channels,
// with the conv-state prefix read as left padding and rolled in place.
// Three entry points follow the three reference kernels:
//   varlen  nanovllm/models/qwen3_5.py:402-473  (prefill over cu_seqlens)
//   decode  nanovllm/models/qwen3_5.py:515-558  (one token, slot pool)
//   padded  nanovllm/models/qwen3_5.py:249-317  ([n, C, T] batches)
// All are HBM-bound.  In varlen and decode each thread owns 8 consecutive
// channels (one 16-byte vector per token row) and slides a 3-token window
// down its token range, so every input is read once (plus a 3-row halo per
// 64-token tile); the padded conv has one kernel per input layout (below).
#include <algorithm>

#include "gdn_common.h"

namespace {

constexpr int kK = 4;        // conv width (Qwen3.5 linear_conv_kernel_dim)
constexpr int kTile = 64;    // tokens per tile
constexpr int kSub = 16;     // tokens per thread
constexpr int kChan = 512;   // channels per tile (64 lanes x 8)

struct Vec8 {
  float v[8];
};

__device__ __forceinline__ Vec8 load8(const uint16_t* p) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint16_t* s = reinterpret_cast<const uint16_t*>(&u);
  Vec8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r.v[i] = gdn::bf2f(s[i]);
  return r;
}

__device__ __forceinline__ void store8(uint16_t* p, const float* v) {
  uint4 u;
  u.x = gdn::f2bf2(v[0], v[1]);
  u.y = gdn::f2bf2(v[2], v[3]);
  u.z = gdn::f2bf2(v[4], v[5]);
  u.w = gdn::f2bf2(v[6], v[7]);
  *reinterpret_cast<uint4*>(p) = u;
}

using gdn::roll_value;
using gdn::silu_acc;

// Finds the (sequence, tile) of flat tile index `tile` given per-sequence
// token counts.  Every sequence owns max(1, ceil(len/64)) tiles (a sequence
// of zero tokens still rolls its state).  One wave scans all sequences.
// Returns false when `tile` is past the last real tile.
__device__ __forceinline__ int64_t tiles_of(int32_t len) {
  return len > 0 ? (static_cast<int64_t>(len) + kTile - 1) / kTile : 1;
}

__device__ bool locate_tile(const int32_t* __restrict__ lens, int n_seqs, int64_t tile,
                            int* seq_out, int64_t* tile_in_seq) {
  __shared__ int s_seq;
  __shared__ long long s_tis;
  if (threadIdx.x == 0) { s_seq = -1; s_tis = 0; }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int per = (n_seqs + 63) / 64;
    const int beg = min(lane * per, n_seqs);
    const int end = min(beg + per, n_seqs);
    long long local = 0;
    for (int r = beg; r < end; ++r) local += tiles_of(lens[r]);
    long long incl = local;  // inclusive wave prefix sum
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const long long o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    const long long excl = incl - local;
    if (tile >= excl && tile < incl) {
      long long acc = excl;
      for (int r = beg; r < end; ++r) {
        const long long nt = tiles_of(lens[r]);
        if (tile < acc + nt) { s_seq = r; s_tis = tile - acc; break; }
        acc += nt;
      }
    }
  }
  __syncthreads();
  *seq_out = s_seq;
  *tile_in_seq = s_tis;
  return s_seq >= 0;
}

// ---------------------------------------------------------------- varlen ----
// grid.x = tile bound (sum of ceil(len/64) <= N/64 + n), grid.y = channel tiles.
// block = 256 threads: lane -> 8 channels, wave -> 16-token sub-tile.
__global__ __launch_bounds__(256) void conv_varlen_kernel(
    const uint16_t* __restrict__ x, int64_t sx_row, uint16_t* __restrict__ state, int64_t ss_seq,
    int64_t ss_ch, const int64_t* __restrict__ ids, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, int key_dim, const int32_t* __restrict__ lens,
    const int32_t* __restrict__ cu_start, int n_seqs, int64_t N, int C) {
  int r;
  int64_t tis;
  if (!locate_tile(lens, n_seqs, blockIdx.x, &r, &tis)) return;
  const int c0 = blockIdx.y * kChan + (threadIdx.x % 64) * 8;
  if (c0 >= C) return;
  const int sub = threadIdx.x / 64;
  const int64_t T = lens[r];
  const int64_t row0 = cu_start[r];
  const int64_t t_beg = tis * kTile + sub * kSub;
  const bool owns_state = (tis == 0 && sub == 0);
  if (t_beg >= T && !owns_state) return;
  const int64_t t_end = min(t_beg + kSub, T);

  // weights for 8 channels
  float wk[8][kK];
  {
    const uint4* wp = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(c0) * kK);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 u = wp[j];
      const uint16_t* s = reinterpret_cast<const uint16_t*>(&u);
#pragma unroll
      for (int i = 0; i < 8; ++i) wk[(j * 8 + i) / kK][(j * 8 + i) % kK] = gdn::bf2f(s[i]);
    }
  }
  const int64_t srow = ids ? ids[r] : r;
  uint16_t* st = state + srow * ss_seq + static_cast<int64_t>(c0) * ss_ch;

  // window: win[0..2] = inputs at t-3, t-2, t-1
  float win[3][8];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int64_t p = t_beg - 3 + j;
    if (p >= 0) {
      const Vec8 v = load8(x + (row0 + p) * sx_row + c0);
#pragma unroll
      for (int i = 0; i < 8; ++i) win[j][i] = v.v[i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t b = st[static_cast<int64_t>(i) * ss_ch + (p + 3)];
        win[j][i] = gdn::bf2f(b);
      }
    }
  }

  const int part = c0 < key_dim ? 0 : (c0 < 2 * key_dim ? 1 : 2);
  const int pw = part < 2 ? key_dim : C - 2 * key_dim;
  uint16_t* yp = y + static_cast<int64_t>(part) * N * key_dim + (c0 - part * key_dim);

#pragma unroll 4
  for (int64_t t = t_beg; t < t_end; ++t) {
    const Vec8 cur = load8(x + (row0 + t) * sx_row + c0);
    float out[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      out[i] = gdn::conv4_silu(win[0][i], win[1][i], win[2][i], cur.v[i], wk[i]);
      win[0][i] = win[1][i];
      win[1][i] = win[2][i];
      win[2][i] = cur.v[i];
    }
    store8(yp + (row0 + t) * pw, out);
  }

  if (owns_state) {
    // new state = raw inputs at positions T-3, T-2, T-1 (old state where < 0)
#pragma unroll
    for (int j = 0; j < kK - 1; ++j) {
      const int64_t p = T - (kK - 1) + j;
      if (p >= 0) {
        const uint4 u = *reinterpret_cast<const uint4*>(x + (row0 + p) * sx_row + c0);
        const uint16_t* s = reinterpret_cast<const uint16_t*>(&u);
#pragma unroll
        for (int i = 0; i < 8; ++i) st[static_cast<int64_t>(i) * ss_ch + j] = roll_value(s[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          st[static_cast<int64_t>(i) * ss_ch + j] = roll_value(st[static_cast<int64_t>(i) * ss_ch + p + (kK - 1)]);
      }
    }
  }
}

// ---------------------------------------------------------------- decode ----
// grid = (ceil(C / 2048), B), block = 256: lane -> 8 channels.
template <bool kVecState>
__global__ __launch_bounds__(256) void conv_decode_kernel(
    const uint16_t* __restrict__ x, int64_t sx_row, uint16_t* __restrict__ pool, int64_t sp_slot,
    int64_t sp_ch, const int64_t* __restrict__ ids, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, int64_t sy_row, int C) {
  const int b = blockIdx.y;
  const int c0 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c0 >= C) return;
  const int64_t slot = ids[b];
  uint16_t* st = pool + slot * sp_slot + static_cast<int64_t>(c0) * sp_ch;
  const uint4 xu = *reinterpret_cast<const uint4*>(x + b * sx_row + c0);
  const uint16_t* xs = reinterpret_cast<const uint16_t*>(&xu);
  uint16_t s[8][3];
  if constexpr (kVecState) {
    uint4 su[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) su[j] = reinterpret_cast<const uint4*>(st)[j];
    const uint16_t* sp = reinterpret_cast<const uint16_t*>(su);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) s[i][j] = sp[i * 3 + j];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) s[i][j] = st[static_cast<int64_t>(i) * sp_ch + j];
  }
  uint16_t wr[8 * kK];
  {
    const uint4* wp = reinterpret_cast<const uint4*>(w + static_cast<int64_t>(c0) * kK);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint4 u = wp[j];
      const uint16_t* q = reinterpret_cast<const uint16_t*>(&u);
#pragma unroll
      for (int i = 0; i < 8; ++i) wr[j * 8 + i] = q[i];
    }
  }
  uint4 yu;
  uint16_t* ys = reinterpret_cast<uint16_t*>(&yu);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float wk[4] = {gdn::bf2f(wr[i * kK]), gdn::bf2f(wr[i * kK + 1]), gdn::bf2f(wr[i * kK + 2]),
                         gdn::bf2f(wr[i * kK + 3])};
    ys[i] = gdn::f2bf(gdn::conv_decode_silu(gdn::bf2f(xs[i]), gdn::bf2f(s[i][0]), gdn::bf2f(s[i][1]),
                                            gdn::bf2f(s[i][2]), wk));
  }
  *reinterpret_cast<uint4*>(y + b * sy_row + c0) = yu;
  // roll: s0 <- s1, s1 <- s2, s2 <- x (bit copies)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s[i][0] = s[i][1];
    s[i][1] = s[i][2];
    s[i][2] = xs[i];
  }
  if constexpr (kVecState) {
    uint4 su[3];
    uint16_t* sp = reinterpret_cast<uint16_t*>(su);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) sp[i * 3 + j] = s[i][j];
#pragma unroll
    for (int j = 0; j < 3; ++j) reinterpret_cast<uint4*>(st)[j] = su[j];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 3; ++j) st[static_cast<int64_t>(i) * sp_ch + j] = s[i][j];
  }
}

// ---------------------------------------------------------------- padded ----
// 8 consecutive bf16 values as fp32, read / written with accesses of V
// elements (V = 8: one 16-byte access, 2: four 4-byte, 1: eight 2-byte); the
// caller guarantees the alignment V implies.
template <int V>
__device__ __forceinline__ void ld8(const uint16_t* p, float (&o)[8]) {
  if constexpr (V == 8) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint16_t* s = reinterpret_cast<const uint16_t*>(&u);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = gdn::bf2f(s[i]);
  } else if constexpr (V == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t u = reinterpret_cast<const uint32_t*>(p)[i];
      o[2 * i] = gdn::bf2f(static_cast<uint16_t>(u));
      o[2 * i + 1] = gdn::bf2f(static_cast<uint16_t>(u >> 16));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = gdn::bf2f(p[i]);
  }
}

template <int V>
__device__ __forceinline__ void st8(uint16_t* p, const uint16_t (&v)[8]) {
  if constexpr (V == 8) {
    uint4 u;
    u.x = v[0] | (static_cast<uint32_t>(v[1]) << 16);
    u.y = v[2] | (static_cast<uint32_t>(v[3]) << 16);
    u.z = v[4] | (static_cast<uint32_t>(v[5]) << 16);
    u.w = v[6] | (static_cast<uint32_t>(v[7]) << 16);
    *reinterpret_cast<uint4*>(p) = u;
  } else if constexpr (V == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      reinterpret_cast<uint32_t*>(p)[i] = v[2 * i] | (static_cast<uint32_t>(v[2 * i + 1]) << 16);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] = v[i];
  }
}

// the conv + SiLU of 8 tokens from the 11-token window xw (tokens t0 - 3 ..
// t0 + 7), in the generic kernel's arithmetic order
__device__ __forceinline__ void conv8(const float (&xw)[11], const float (&w4)[kK], uint16_t (&out)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kK; ++i) acc += xw[k + i] * w4[i];
    out[k] = gdn::f2bf(silu_acc(acc));
  }
}

// Padded conv, time-contiguous input (token stride 1): one thread per
// (sequence, channel, 8 consecutive tokens), no LDS.  The 3-token halo comes
// from the previous 8 tokens (the neighbouring lane's load: a cache hit), or
// from the conv state for the first 8.  The thread of the first 8 tokens is
// the only reader of a channel's old state, and writes the new one.
// grid = ceil(n * C * ceil(T / 8) / 256); block = 256.
template <int V>
__global__ __launch_bounds__(256) void conv_padded_tfast_kernel(
    const uint16_t* __restrict__ x, int64_t sx_n, int64_t sx_c, uint16_t* __restrict__ state, int64_t ss_n,
    int64_t ss_c, const uint16_t* __restrict__ w, uint16_t* __restrict__ y, const int32_t* __restrict__ endp,
    int C, int T, int G, int total) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= total) return;
  const int row = idx / G, g = idx - row * G;  // row = n * C + c
  const int n = row / C, c = row - n * C;
  const int t0 = 8 * g;
  const uint16_t* xc = x + static_cast<int64_t>(n) * sx_n + static_cast<int64_t>(c) * sx_c;
  uint16_t* sc = state + static_cast<int64_t>(n) * ss_n + static_cast<int64_t>(c) * ss_c;
  float w4[kK];
#pragma unroll
  for (int i = 0; i < kK; ++i) w4[i] = gdn::bf2f(w[static_cast<int64_t>(c) * kK + i]);
  float xw[11];
  float s_old[kK - 1] = {0.0f, 0.0f, 0.0f};
  if (g == 0) {
#pragma unroll
    for (int j = 0; j < kK - 1; ++j) s_old[j] = gdn::bf2f(sc[j]);
#pragma unroll
    for (int j = 0; j < 3; ++j) xw[j] = s_old[j];
  } else {
    float prev[8];
    ld8<V>(xc + t0 - 8, prev);
#pragma unroll
    for (int j = 0; j < 3; ++j) xw[j] = prev[5 + j];
  }
  float cur[8];
  if (t0 + 8 <= T) {
    ld8<V>(xc + t0, cur);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) cur[i] = t0 + i < T ? gdn::bf2f(xc[t0 + i]) : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) xw[3 + i] = cur[i];
  uint16_t out[8];
  conv8(xw, w4, out);
  uint16_t* yr = y + static_cast<int64_t>(row) * T + t0;
  if (t0 + 8 <= T) {
    st8<V>(yr, out);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (t0 + i < T) yr[i] = out[i];
  }
  if (g == 0) {
    const int e = endp[n];
    if (e >= 0) {
#pragma unroll
      for (int j = 0; j < kK - 1; ++j) {
        const int p = e - (kK - 1) + j;
        // the old state is exact in fp32 (bf16 -> fp32 -> bf16 round trip)
        const uint16_t bits = p < 0 ? gdn::f2bf(s_old[p + kK - 1]) : p < T ? xc[p] : static_cast<uint16_t>(0);
        sc[j] = roll_value(bits);
      }
    }
  }
}

// Padded conv, channel-stride-1 input (the reference's [n, T, C] rows): the
// 64-channel x 67-token window is staged through LDS with loads of VL
// channels along each token row (the transpose), then thread (channel tid / 4,
// 16 tokens) computes its outputs and writes them along T with accesses of
// VS tokens.  Row stride 69 floats: both the staging writes and the window
// reads are free of bank conflicts.
// grid = (ceil(T / 64), ceil(C / 64), n); block = 256.
template <int VL, int VS>
__global__ __launch_bounds__(256) void conv_padded_cfast_kernel(
    const uint16_t* __restrict__ x, int64_t sx_n, int64_t sx_t, uint16_t* __restrict__ state, int64_t ss_n,
    int64_t ss_c, const uint16_t* __restrict__ w, uint16_t* __restrict__ y, const int32_t* __restrict__ endp,
    int C, int T) {
  __shared__ float tile[64][69];
  const int n = blockIdx.z;
  const int cb = blockIdx.y * 64;
  const int t0 = blockIdx.x * kTile;
  const uint16_t* xn = x + static_cast<int64_t>(n) * sx_n;
  uint16_t* sn = state + static_cast<int64_t>(n) * ss_n;
  for (int e = threadIdx.x; e < 8 * (kTile + 3); e += 256) {
    const int j = e >> 3, q = e & 7;
    const int p = t0 - 3 + j;
    const int c0 = cb + 8 * q;
    float v[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (c0 < C) {  // C % 8 == 0: all 8 channels exist
      if (p >= 0 && p < T) {
        ld8<VL>(xn + static_cast<int64_t>(p) * sx_t + c0, v);
      } else if (p < 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = gdn::bf2f(sn[static_cast<int64_t>(c0 + i) * ss_c + (p + 3)]);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) tile[8 * q + i][j] = v[i];
  }
  __syncthreads();
  const int c = threadIdx.x >> 2, tg = threadIdx.x & 3;
  const int cc = cb + c;
  if (cc < C) {
    float w4[kK];
#pragma unroll
    for (int i = 0; i < kK; ++i) w4[i] = gdn::bf2f(w[static_cast<int64_t>(cc) * kK + i]);
    uint16_t* yr = y + (static_cast<int64_t>(n) * C + cc) * T;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int tl = 16 * tg + 8 * h;  // first of 8 tokens, tile-relative
      float xw[11];
#pragma unroll
      for (int i = 0; i < 11; ++i) xw[i] = tile[c][tl + i];
      uint16_t out[8];
      conv8(xw, w4, out);
      const int t = t0 + tl;
      if (t + 8 <= T) {
        st8<VS>(yr + t, out);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (t + i < T) yr[t + i] = out[i];
      }
    }
  }
  // state write-back by the first token tile (the only reader of the old
  // state), from the staged old state
  if (blockIdx.x == 0) {
    const int e = endp[n];
    if (e >= 0) {
      for (int idx = threadIdx.x; idx < 64 * (kK - 1); idx += 256) {
        const int ch = idx / (kK - 1);
        const int j = idx % (kK - 1);
        const int ccw = cb + ch;
        if (ccw >= C) continue;
        const int p = e - (kK - 1) + j;
        uint16_t bits;
        if (p < 0) bits = gdn::f2bf(tile[ch][p + 3]);
        else bits = p < T ? xn[static_cast<int64_t>(p) * sx_t + ccw] : static_cast<uint16_t>(0);
        sn[static_cast<int64_t>(ccw) * ss_c + j] = roll_value(bits);
      }
    }
  }
}

// Any other strides: element by element through LDS.
// grid = (ceil(T/64), ceil(C/64), n); block = 256.  The x tile (64 channels x
// 67 tokens incl. halo) is staged in LDS so both the strided input and the
// T-contiguous output are accessed along their unit-stride dimension.
__global__ __launch_bounds__(256) void conv_padded_kernel(
    const uint16_t* __restrict__ x, int64_t sx_n, int64_t sx_c, int64_t sx_t,
    uint16_t* __restrict__ state, int64_t ss_n, int64_t ss_c, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, const int32_t* __restrict__ endp, int C, int T, int chan_fast) {
  __shared__ float tile[64][kTile + 3 + 1];
  const int n = blockIdx.z;
  const int cb = blockIdx.y * 64;
  const int t0 = blockIdx.x * kTile;
  const uint16_t* xn = x + static_cast<int64_t>(n) * sx_n;
  uint16_t* sn = state + static_cast<int64_t>(n) * ss_n;
  // stage inputs at positions t0-3 .. t0+63 (state for p < 0, zero past T)
  for (int e = threadIdx.x; e < 64 * (kTile + 3); e += 256) {
    int c, j;
    if (chan_fast) { c = e % 64; j = e / 64; } else { j = e % (kTile + 3); c = e / (kTile + 3); }
    const int cc = cb + c;
    const int p = t0 - 3 + j;
    float val = 0.0f;
    if (cc < C) {
      if (p >= 0 && p < T) val = gdn::bf2f(xn[static_cast<int64_t>(cc) * sx_c + static_cast<int64_t>(p) * sx_t]);
      else if (p < 0) val = gdn::bf2f(sn[static_cast<int64_t>(cc) * ss_c + (p + 3)]);
    }
    tile[c][j] = val;
  }
  __syncthreads();
  // outputs: thread -> (token = tid % 64, channel group)
  const int tl = threadIdx.x % 64;
  const int t = t0 + tl;
  for (int c = threadIdx.x / 64; c < 64; c += 4) {
    const int cc = cb + c;
    if (cc >= C || t >= T) continue;
    const uint16_t* wp = w + static_cast<int64_t>(cc) * kK;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kK; ++i) acc += tile[c][tl + i] * gdn::bf2f(wp[i]);
    y[(static_cast<int64_t>(n) * C + cc) * T + t] = gdn::f2bf(silu_acc(acc));
  }
  // state writeback by the first token tile (the only reader of the old state)
  if (blockIdx.x == 0) {
    const int e = endp[n];
    if (e >= 0) {
      for (int idx = threadIdx.x; idx < 64 * (kK - 1); idx += 256) {
        const int c = idx / (kK - 1);
        const int j = idx % (kK - 1);
        const int cc = cb + c;
        if (cc >= C) continue;
        const int p = e - (kK - 1) + j;
        uint16_t bits;
        if (p >= 0) bits = xn[static_cast<int64_t>(cc) * sx_c + static_cast<int64_t>(p) * sx_t];
        else bits = gdn::f2bf(tile[c][p + 3]);  // old state, staged above (p + 3 < 3)
        // the staged old state is exact (bf16 -> fp32 -> bf16 round trip)
        sn[static_cast<int64_t>(cc) * ss_c + j] = roll_value(bits);
      }
    }
  }
}

}  // namespace

extern "C" int gdn_conv_varlen(const uint16_t* x, int64_t sx_row, uint16_t* state, int64_t ss_seq,
                               int64_t ss_ch, const int64_t* ids, const uint16_t* w, uint16_t* y,
                               int key_dim, const int32_t* lens, const int32_t* cu_start,
                               int n_seqs, int64_t N, int C, int K, void* stream) {
  if (K != kK) return GDN_ERR_UNSUPPORTED;
  if (n_seqs < 0 || N < 0 || C <= 0 || C % 8 || key_dim <= 0 || key_dim % 8 ||
      2 * key_dim >= C || (C - 2 * key_dim) % 8 || sx_row % 8)
    return GDN_ERR_INVALID_ARG;
  if (n_seqs == 0) return GDN_OK;
  if (!x || !state || !w || !y || !lens || !cu_start) return GDN_ERR_INVALID_ARG;
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
      reinterpret_cast<uintptr_t>(y) % 16 || (N * key_dim) % 8)
    return GDN_ERR_INVALID_ARG;
  const int64_t tiles = (N + kTile - 1) / kTile + n_seqs;
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>((C + kChan - 1) / kChan));
  conv_varlen_kernel<<<grid, dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      x, sx_row, state, ss_seq, ss_ch, ids, w, y, key_dim, lens, cu_start, n_seqs, N, C);
  return gdn_launch_status();
}

extern "C" int gdn_conv_decode(const uint16_t* x, int64_t sx_row, uint16_t* pool, int64_t sp_slot,
                               int64_t sp_ch, const int64_t* ids, const uint16_t* w, uint16_t* y,
                               int64_t sy_row, int B, int C, int K, void* stream) {
  if (K != kK) return GDN_ERR_UNSUPPORTED;
  if (B < 0 || C <= 0 || C % 8 || sx_row % 8 || sy_row % 8) return GDN_ERR_INVALID_ARG;
  if (B == 0) return GDN_OK;
  if (!x || !pool || !ids || !w || !y) return GDN_ERR_INVALID_ARG;
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(w) % 16 ||
      reinterpret_cast<uintptr_t>(y) % 16)
    return GDN_ERR_INVALID_ARG;
  const bool vec = sp_ch == kK - 1 && sp_slot % 8 == 0 && reinterpret_cast<uintptr_t>(pool) % 16 == 0;
  const dim3 grid(static_cast<unsigned>((C + 2047) / 2048), static_cast<unsigned>(B));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec)
    conv_decode_kernel<true><<<grid, dim3(256), 0, s>>>(x, sx_row, pool, sp_slot, sp_ch, ids, w, y, sy_row, C);
  else
    conv_decode_kernel<false><<<grid, dim3(256), 0, s>>>(x, sx_row, pool, sp_slot, sp_ch, ids, w, y, sy_row, C);
  return gdn_launch_status();
}

extern "C" int gdn_conv_padded(const uint16_t* x, int64_t sx_n, int64_t sx_c, int64_t sx_t,
                               uint16_t* state, int64_t ss_n, int64_t ss_c, const uint16_t* w,
                               uint16_t* y, const int32_t* endp, int n, int C, int T, int K,
                               void* stream) {
  if (K != kK) return GDN_ERR_UNSUPPORTED;
  if (n < 0 || C <= 0 || T < 0) return GDN_ERR_INVALID_ARG;
  if (n == 0 || T == 0) return GDN_OK;
  if (!x || !state || !w || !y || !endp) return GDN_ERR_INVALID_ARG;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const uintptr_t xa = reinterpret_cast<uintptr_t>(x), ya = reinterpret_cast<uintptr_t>(y);
  // widest access that every row start allows: 8 elements (16 B), 2 (4 B) or 1
  auto width = [](int64_t stride, uintptr_t base) {
    return stride % 8 == 0 && base % 16 == 0 ? 8 : stride % 2 == 0 && base % 4 == 0 ? 2 : 1;
  };
  const int vs = width(T, ya);  // output rows [n, C, T]
  const int64_t G = (T + 7) / 8;
  if (sx_t == 1 && sx_n >= 0 && sx_c >= 0 && static_cast<int64_t>(n) * C * G < (1LL << 31)) {
    const int total = static_cast<int>(static_cast<int64_t>(n) * C * G);
    const int v = std::min(width(sx_c, xa), vs) == 8 && sx_n % 8 == 0 ? 8
                : std::min(width(sx_c, xa), vs) >= 2 && sx_n % 2 == 0 ? 2 : 1;
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    if (v == 8)
      conv_padded_tfast_kernel<8><<<grid, dim3(256), 0, st>>>(x, sx_n, sx_c, state, ss_n, ss_c, w, y, endp, C, T,
                                                              static_cast<int>(G), total);
    else if (v == 2)
      conv_padded_tfast_kernel<2><<<grid, dim3(256), 0, st>>>(x, sx_n, sx_c, state, ss_n, ss_c, w, y, endp, C, T,
                                                              static_cast<int>(G), total);
    else
      conv_padded_tfast_kernel<1><<<grid, dim3(256), 0, st>>>(x, sx_n, sx_c, state, ss_n, ss_c, w, y, endp, C, T,
                                                              static_cast<int>(G), total);
    return gdn_launch_status();
  }
  const dim3 grid(static_cast<unsigned>((T + kTile - 1) / kTile), static_cast<unsigned>((C + 63) / 64),
                  static_cast<unsigned>(n));
  if (sx_c == 1 && C % 8 == 0 && sx_n >= 0 && sx_t >= 0) {
    const int vl = width(sx_t, xa) == 8 && sx_n % 8 == 0 ? 8 : width(sx_t, xa) >= 2 && sx_n % 2 == 0 ? 2 : 1;
#define GDN_CFAST(VL, VS)                                                                                   \
  conv_padded_cfast_kernel<VL, VS><<<grid, dim3(256), 0, st>>>(x, sx_n, sx_t, state, ss_n, ss_c, w, y, endp, C, T)
    if (vl == 8) {
      if (vs == 8) GDN_CFAST(8, 8); else if (vs == 2) GDN_CFAST(8, 2); else GDN_CFAST(8, 1);
    } else if (vl == 2) {
      if (vs == 8) GDN_CFAST(2, 8); else if (vs == 2) GDN_CFAST(2, 2); else GDN_CFAST(2, 1);
    } else {
      if (vs == 8) GDN_CFAST(1, 8); else if (vs == 2) GDN_CFAST(1, 2); else GDN_CFAST(1, 1);
    }
#undef GDN_CFAST
    return gdn_launch_status();
  }
  const int chan_fast = (sx_c == 1) || (sx_t != 1 && llabs(sx_c) <= llabs(sx_t));
  conv_padded_kernel<<<grid, dim3(256), 0, st>>>(x, sx_n, sx_c, sx_t, state, ss_n, ss_c, w, y, endp, C, T,
                                                 chan_fast);
  return gdn_launch_status();
}
