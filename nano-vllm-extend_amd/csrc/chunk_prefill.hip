// Chunked gated delta rule over packed varlen sequences, chunk size 64.
//
// Per chunk (rows t, s in [0, 64); G = inclusive cumsum of g in the chunk,
// gamma = G[63]; k^, q^ = L2-normalised rows; the algorithm of the torch
// port at nanovllm/models/qwen3_5.py:152-227):
//   L    = strict_lower( beta_t k^_t.k^_s e^{G_t-G_s} )
//   T    = (I + L)^-1                       (the reference's forward substitution)
//   W    = T diag(beta e^G) K^,   U = T diag(beta) V
//   Vn   = U - W S
//   O    = diag(scale e^G) Q^ S + A Vn,   A = lower_incl( scale q^_t.k^_s e^{G_t-G_s} )
//   S   <- e^gamma S + K^T diag(e^{gamma-G}) Vn
//
// Two kernels.
//   chunk_prep_kernel: one workgroup per (chunk, value head), all chunks in
//     parallel.  Everything that needs only the chunk's own q, k, g, beta:
//     the row norms, K K^T, Q K^T, the triangular inverse T (fp32), and it
//     writes a 26 KiB record: T diag(beta e^G), T diag(beta) and A as fp16
//     64x64 tiles plus the per-token scales.
//   chunk_state_kernel: one workgroup per (sequence, value head, block of 64
//     value columns), persistent over the sequence's chunks.  Producer waves
//     stage the next chunk (raw q rows, K^ and V transposed, all fp16; the
//     record's tiles; W = T' K^ by MFMA) into a double-buffered LDS stage
//     while two chain waves run the state-dependent products of the current
//     chunk with their 128 x 32 slice of S in registers.
//
// Numerics.  Every state-path product runs on the fp16 matrix cores
// (v_mfma_f32_32x32x16_f16, fp32 accumulation) with one pass: fp16 keeps 11
// significant bits, and a CPU simulation of this scheme against an fp64
// recurrence gives output mean-rel ~3e-4 and state rel ~2.6e-4 at the
// slow decays of trained checkpoints (bf16 single-pass operands give
// ~2e-3).  K is L2-normalised (in fp32) before its fp16 conversion, so its
// operands lie in [-1, 1]; raw q, v and T, S, Vn must stay below the fp16
// maximum (65504), far above any trained model's range (1/||q|| is applied
// to the output rows in fp32).  q k^T and k k^T of the
// prep kernel use the raw bf16 rows (exact operands); T is computed in fp32.
//
// Layouts.  32x32x16 MFMA fragments: A lane l holds row (l & 31), B lane l
// column (l & 31), each with 8 contraction values in lane group g = l >> 5;
// the C tile gives lane l column (l & 31) and rows 8i + 4g + r in acc[4i+r].
// Two adjacent C rows-of-8 blocks (i = 2h, 2h + 1) hold the 8 contraction
// values a B (or A) operand needs for 16 consecutive rows, in the order
// {16h + 4g + r, 16h + 8 + 4g + r}.  qswap() (swap quads 1 and 2 of every
// 16-block) maps that order onto 8 contiguous indices 16h + 8g + 0..7, so:
//   * the state's row positions p hold key qswap(p): W and Q^ are then read
//     as plain rows (16 contiguous bytes per lane);
//   * the token index of K^T, V^T and of the columns of T', T'', A is stored
//     in position order: position p holds token qswap(p), which is the order
//     in which the C tiles of the transposes deliver them.
// fp16 tiles in LDS and in the record are row-major with 16-byte granules
// XOR-swizzled by row (swz), so 16 lanes reading one granule column of 16
// rows hit 16 distinct bank groups.
#include "gdn_common.h"

namespace {

using gdn::f32x4_t;
using gdn::s16x8_t;

typedef _Float16 h16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kC = 64;   // chunk size (tokens)
constexpr int kCB = 64;  // value columns per state workgroup

__device__ __forceinline__ int64_t chunks_of(int64_t len) { return (len + kC - 1) / kC; }

// swap quads 1 and 2 of each 16-block (an involution)
__device__ __forceinline__ int qswap(int p) { return (p & ~12) | ((p & 4) << 1) | ((p & 8) >> 1); }

// element offset of (r, c) in a row-major fp16 tile with RL elements per row
template <int RL>
__device__ __forceinline__ int swz(int r, int c) {
  constexpr int G = RL / 8;  // 16-byte granules per row: 8 or 16
  const int x = (r / (16 / G)) & (G - 1);
  return r * RL + (((c >> 3) ^ x) << 3) + (c & 7);
}

__device__ __forceinline__ float lo_half(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_half(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// two fp32 -> fp16x2, round to nearest even
__device__ __forceinline__ uint32_t f2h2(float a, float b) {
  const gdn::f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h16x2_t));
}

// elements [o, o + 8) of a C tile -> fp16 operand fragment
template <int O>
__device__ __forceinline__ h16x8_t pack_h8(const f32x16_t& a) {
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = f2h2(a[O + 2 * p], a[O + 2 * p + 1]);
  return __builtin_bit_cast(h16x8_t, r);
}

__device__ __forceinline__ f32x16_t mfma32(const h16x8_t& a, const h16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ h16x8_t ld_h8(const uint16_t* base, int off) {
  return *reinterpret_cast<const h16x8_t*>(base + off);
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- record of one (chunk, value head), byte offsets ----
// T' = T diag(beta e^G / ||k||), T'' = T diag(beta) and A are zero above the
// diagonal 32x32 blocks; each is stored as its three nonzero 32x32 blocks
// (0,0), (1,0), (1,1) (block index = row block + column block), fp16, 32-wide
// rows with swizzled granules (swz<32>), columns in position order (position
// p holds token qswap(p)).
//   TW  [3][32][32] fp16   T'
//   TB  [3][32][32] fp16   T''
//   AQ  [3][32][32] fp16   A
//   VEC fp32 [256]         cQ[64] = scale e^{G_t} / ||q_t||,
//                          cK[64] = e^{gamma - G_t} / ||k_t|| (0 past the sequence end),
//                          e^gamma
// The tiles are stored exactly as the state kernel's LDS holds them, so it
// copies them linearly.
struct Rec {
  static constexpr int TW = 0;
  static constexpr int TB = 6144;
  static constexpr int AQ = 12288;
  static constexpr int VEC = 18432;
  static constexpr int BYTES = 19456;
};

// element offset of (row, col) of a 64x64 block-lower-triangular tile stored
// as its three nonzero 32x32 blocks (col / 32 <= row / 32)
__device__ __forceinline__ int tri_off(int row, int col) {
  return ((row >> 5) + (col >> 5)) * 1024 + swz<32>(row & 31, col & 31);
}

// Flat chunk index -> (sequence, chunk within it), by one wave scanning the
// per-sequence chunk counts.  Returns false past the last chunk.
__device__ bool locate_chunk(const int64_t* __restrict__ cu, int n_seqs, int64_t c, int* seq_out,
                             int64_t* j_out) {
  __shared__ int s_seq;
  __shared__ long long s_j;
  if (threadIdx.x == 0) { s_seq = -1; s_j = 0; }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int per = (n_seqs + 63) / 64;
    const int beg = min(lane * per, n_seqs);
    const int end = min(beg + per, n_seqs);
    long long local = 0;
    for (int r = beg; r < end; ++r) local += chunks_of(cu[r + 1] - cu[r]);
    long long incl = local;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const long long o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    const long long excl = incl - local;
    if (c >= excl && c < incl) {
      long long acc = excl;
      for (int r = beg; r < end; ++r) {
        const long long nc = chunks_of(cu[r + 1] - cu[r]);
        if (c < acc + nc) { s_seq = r; s_j = c - acc; break; }
        acc += nc;
      }
    }
  }
  __syncthreads();
  *seq_out = s_seq;
  *j_out = s_j;
  return s_seq >= 0;
}

// ============================================================= prep kernel ==
// acc += A(16x16) B(16x16), fp32 operands in LDS, fp32 matrix cores.
__device__ __forceinline__ f32x4_t mm16_f32(f32x4_t acc, const float* A, int lda, const float* B, int ldb, int lane) {
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    acc = gdn::mfma16x16x4f32(A[lr * lda + 4 * kk + lg], B[(4 * kk + lg) * ldb + lr], acc);
  return acc;
}

constexpr int kTileLd = 20;  // row stride (floats) of a packed fp32 16x16 tile

__device__ __forceinline__ void st16_f32(float* Cp, const f32x4_t& acc, float alpha, int lane) {
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) Cp[(4 * lg + i) * kTileLd + lr] = alpha * acc[i];
}

__device__ __forceinline__ f32x4_t ld16_f32(const float* Cp, int lane) {
  const int lr = lane & 15, lg = lane >> 4;
  f32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = Cp[(4 * lg + i) * kTileLd + lr];
  return r;
}

// lower-triangular 16x16 tile index j in [0, 10) <-> (mt, nt), mt >= nt
__device__ __forceinline__ void tri_tile(int j, int& mt, int& nt) {
  mt = j >= 6 ? 3 : (j >= 3 ? 2 : (j >= 1 ? 1 : 0));
  nt = j - (mt * (mt + 1)) / 2;
}
__device__ __forceinline__ int tix(int mt, int nt) { return (mt * (mt + 1)) / 2 + nt; }

template <int D>
struct __align__(16) PrepSmem {
  uint16_t Kr[kC][D + 8];         // raw bf16 K rows
  float Lp[10][16][kTileLd];      // lower tiles of L
  float Tp[10][16][kTileLd];      // lower tiles of T = (I + L)^-1
  float scr[4][16][kTileLd];      // per-wave scratch of the solve
  float G[kC], bt[kC], rk[kC], rq[kC], ssk[kC], ssq[kC], cw[kC];
};

// Row t, token quad Q (tokens 4Q..4Q+3) of T, times c[s]: 4 floats.
__device__ __forceinline__ float4 t_quad(const float (*Tp)[16][kTileLd], const float* c, int t, int Q) {
  const int mt = t >> 4, st = Q >> 2;
  if (st > mt) return make_float4(0.f, 0.f, 0.f, 0.f);
  const float4 r = *reinterpret_cast<const float4*>(&Tp[tix(mt, st)][t & 15][(Q & 3) * 4]);
  const float4 cc = *reinterpret_cast<const float4*>(&c[4 * Q]);
  return make_float4(r.x * cc.x, r.y * cc.y, r.z * cc.z, r.w * cc.w);
}

// quad index (4 tokens) of the tokens at positions [4P, 4P + 4)
__device__ __forceinline__ int quad_of_pos(int P) { return qswap(4 * P) >> 2; }

// grid = 8 * ceil(nc_bound * Hv / 8); block = 256.  One workgroup per
// (chunk, value head); writes the chunk's record.
template <int D>
__global__ __launch_bounds__(256) void chunk_prep_kernel(
    const uint16_t* __restrict__ q, int64_t sq, const uint16_t* __restrict__ k, int64_t sk,
    const float* __restrict__ g, const uint16_t* __restrict__ beta, const int64_t* __restrict__ cu,
    int n_seqs, int64_t nc_bound, int Hk, int Hv, float scale, int l2norm, uint8_t* __restrict__ ws) {
  constexpr int NW = 4;
  constexpr int NT = 64 * NW;
  constexpr int KTD = D / 32;
  constexpr int SEG = D / 8;            // 16-byte segments per row
  constexpr int NSEG1 = kC * SEG / NT;  // row segments per thread
  static_assert(kC * SEG % NT == 0 && NT % SEG == 0, "segment tiling");
  __shared__ PrepSmem<D> sm;

  const int64_t wi = gdn::xcd_remap(blockIdx.x, nc_bound * Hv);
  if (wi < 0) return;
  const int h = static_cast<int>(wi % Hv);
  const int64_t cidx = wi / Hv;
  int r;
  int64_t jc;
  if (!locate_chunk(cu, n_seqs, cidx, &r, &jc)) return;
  const int64_t tok0 = cu[r] + jc * kC;
  const int len = static_cast<int>(min<int64_t>(kC, cu[r + 1] - tok0));
  const int kh = h / (Hv / Hk);
  const uint16_t* qh = q + static_cast<int64_t>(kh) * D;
  const uint16_t* kh_ = k + static_cast<int64_t>(kh) * D;
  uint8_t* rec = ws + (cidx * Hv + h) * Rec::BYTES;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // Waves 1..3 form the A blocks b = wave - 1 and wave + 2 later on; their q
  // rows (B operands) are loaded now so the loads overlap the whole first half.
  s16x8_t qpre[2][KTD];
  if (wave > 0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = wave - 1 + 3 * u;
      const int mt = b < 2 ? b : 2 + ((b - 2) >> 1);
      const uint16_t* qr = qh + (tok0 + min(16 * mt + lr, len - 1)) * sq + 8 * lg;
#pragma unroll
      for (int kk = 0; kk < KTD; ++kk) qpre[u][kk] = *reinterpret_cast<const s16x8_t*>(qr + 32 * kk);
    }
  }

  // ---- phase 1: K rows, row norms of K and Q, gates ----
#pragma unroll
  for (int j = 0; j < NSEG1; ++j) {
    const int e = tid + NT * j;
    const int t = e / SEG, c8 = e % SEG;
    const int64_t row = tok0 + min(t, len - 1);
    s16x8_t kv8 = *reinterpret_cast<const s16x8_t*>(kh_ + row * sk + c8 * 8);
    s16x8_t qv8 = *reinterpret_cast<const s16x8_t*>(qh + row * sq + c8 * 8);
    if (t >= len) {
      kv8 = s16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      qv8 = kv8;
    }
    *reinterpret_cast<s16x8_t*>(&sm.Kr[t][c8 * 8]) = kv8;
    float ks = 0.f, qs = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float kf = gdn::bf2f(static_cast<uint16_t>(kv8[i]));
      const float qf = gdn::bf2f(static_cast<uint16_t>(qv8[i]));
      ks += kf * kf;
      qs += qf * qf;
    }
#pragma unroll
    for (int m = SEG / 2; m >= 1; m >>= 1) {
      ks += __shfl_xor(ks, m, 64);
      qs += __shfl_xor(qs, m, 64);
    }
    if (c8 == 0) {
      sm.ssk[t] = ks;
      sm.ssq[t] = qs;
    }
  }
  if (wave == 0) {
    float gv = 0.f, bv = 0.f;
    if (lane < len) {
      const int64_t gi = (tok0 + lane) * Hv + h;
      gv = g[gi];
      bv = gdn::bf2f(beta[gi]);
    }
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float o_ = __shfl_up(gv, d, 64);
      if (lane >= d) gv += o_;
    }
    sm.G[lane] = gv;
    sm.bt[lane] = bv;
  }
  __syncthreads();
  if (tid < kC) {
    const int t = tid;
    // rk = 0 past the sequence end: cK and T' then clear those key tokens
    const float rk = t < len ? (l2norm ? rsqrtf(sm.ssk[t] + 1e-6f) : 1.0f) : 0.f;
    const float rq = l2norm ? rsqrtf(sm.ssq[t] + 1e-6f) : 1.0f;
    const float Gt = sm.G[t];
    const float Gl = sm.G[kC - 1];
    sm.rk[t] = rk;
    sm.rq[t] = rq;
    sm.cw[t] = sm.bt[t] * rk * expf(Gt);
    float* vec = reinterpret_cast<float*>(rec + Rec::VEC);
    vec[t] = rq * scale * expf(Gt);
    vec[kC + t] = rk * expf(Gl - Gt);
    if (t == 0) vec[2 * kC] = expf(Gl);
  }
  __syncthreads();

  // ---- phase 2a: K K^T -> L (fp32 lower tiles) ----
  for (int j = wave; j < 10; j += NW) {
    int mt, nt;
    tri_tile(j, mt, nt);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KTD; ++kk) {
      const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.Kr[16 * mt + lr][32 * kk + 8 * lg]);
      const s16x8_t b8 = *reinterpret_cast<const s16x8_t*>(&sm.Kr[16 * nt + lr][32 * kk + 8 * lg]);
      acc = gdn::mfma16x16x32(a8, b8, acc);
    }
    const int s = 16 * nt + lr;
    const float rks = sm.rk[s];
    const float Gs = sm.G[s];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * mt + 4 * lg + i;
      sm.Lp[j][4 * lg + i][lr] = s < t ? acc[i] * sm.bt[t] * sm.rk[t] * rks * __expf(sm.G[t] - Gs) : 0.f;
    }
  }
  __syncthreads();

  // ---- phase 2b: wave 0 inverts the diagonal blocks; the other waves form
  //      A = lower_incl(scale q^.k^ e^{G_t - G_s}) and write it to the record ----
  if (wave == 0) {
    const int bb = lane >> 4, c = lane & 15;
    const int dt = tix(bb, bb);
    float x[16];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float4* lrow = reinterpret_cast<const float4*>(&sm.Lp[dt][rr][0]);
      float lv[16];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 f = lrow[q4];
        lv[4 * q4] = f.x; lv[4 * q4 + 1] = f.y; lv[4 * q4 + 2] = f.z; lv[4 * q4 + 3] = f.w;
      }
      float acc = rr == c ? 1.f : 0.f;
#pragma unroll
      for (int jj = 0; jj < rr; ++jj) acc -= lv[jj] * x[jj];
      x[rr] = acc;
    }
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) sm.Tp[dt][rr][c] = x[rr];
  } else {
    // blocks (mt, kt): query rows 16 mt.., key tokens 32 kt.. with 32 kt <= 16 mt + 15
    uint16_t* arec = reinterpret_cast<uint16_t*>(rec + Rec::AQ);
    static_assert(NW == 4, "waves 1..3 take two A blocks each");
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int b = wave - 1 + 3 * u;
      const int mt = b < 2 ? b : 2 + ((b - 2) >> 1);
      const int kt = b < 2 ? 0 : ((b - 2) & 1);
      const int t = 16 * mt + lr;  // the lane's query token (C column)
      const s16x8_t* qb = qpre[u];
      const float qscale = sm.rq[t] * scale;
      const float Gt = sm.G[t];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ns = 2 * kt + half;  // key-token tile
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        if (ns <= mt) {
#pragma unroll
          for (int kk = 0; kk < KTD; ++kk) {
            const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.Kr[16 * ns + lr][32 * kk + 8 * lg]);
            acc = gdn::mfma16x16x32(a8, qb[kk], acc);
          }
        }
        float a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int s = 16 * ns + 4 * lg + i;
          a[i] = (s <= t && t < len) ? acc[i] * qscale * sm.rk[s] * __expf(Gt - sm.G[s]) : 0.f;
        }
        // tokens 16 ns + 4 lg .. + 3 sit at the positions of quad qswap
        const int pos = qswap(16 * ns + 4 * lg);
        uint2 pk;
        pk.x = f2h2(a[0], a[1]);
        pk.y = f2h2(a[2], a[3]);
        *reinterpret_cast<uint2*>(&arec[tri_off(t, pos)]) = pk;
      }
    }
  }
  __syncthreads();
  // first sub-diagonal: T(j+1, j) = -T(j+1,j+1) L(j+1,j) T(j,j)
  if (wave < 3) {
    const int j = wave, i = j + 1;
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(i, j)][0][0], kTileLd, &sm.Tp[tix(j, j)][0][0], kTileLd, lane);
    st16_f32(&sm.scr[wave][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(i, i)][0][0], kTileLd, &sm.scr[wave][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(i, j)][0][0], t2, -1.f, lane);
  } else {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(3, 0)][0][0], kTileLd, &sm.Tp[tix(0, 0)][0][0], kTileLd, lane);  // L30 T00
    st16_f32(&sm.scr[3][0][0], p, 1.f, lane);
  }
  __syncthreads();
  // second sub-diagonal: T20, T31; partial sum for T30
  if (wave == 0) {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(2, 0)][0][0], kTileLd, &sm.Tp[tix(0, 0)][0][0], kTileLd, lane);  // L20 T00
    p = mm16_f32(p, &sm.Lp[tix(2, 1)][0][0], kTileLd, &sm.Tp[tix(1, 0)][0][0], kTileLd, lane);  // L21 T10
    st16_f32(&sm.scr[0][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(2, 2)][0][0], kTileLd, &sm.scr[0][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(2, 0)][0][0], t2, -1.f, lane);
  } else if (wave == 1) {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(3, 1)][0][0], kTileLd, &sm.Tp[tix(1, 1)][0][0], kTileLd, lane);  // L31 T11
    p = mm16_f32(p, &sm.Lp[tix(3, 2)][0][0], kTileLd, &sm.Tp[tix(2, 1)][0][0], kTileLd, lane);  // L32 T21
    st16_f32(&sm.scr[1][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(3, 3)][0][0], kTileLd, &sm.scr[1][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(3, 1)][0][0], t2, -1.f, lane);
  } else if (wave == 3) {
    f32x4_t p = ld16_f32(&sm.scr[3][0][0], lane);
    p = mm16_f32(p, &sm.Lp[tix(3, 1)][0][0], kTileLd, &sm.Tp[tix(1, 0)][0][0], kTileLd, lane);  // + L31 T10
    st16_f32(&sm.scr[3][0][0], p, 1.f, lane);
  }
  __syncthreads();
  // third sub-diagonal: T30
  if (wave == 3) {
    f32x4_t p = ld16_f32(&sm.scr[3][0][0], lane);
    p = mm16_f32(p, &sm.Lp[tix(3, 2)][0][0], kTileLd, &sm.Tp[tix(2, 0)][0][0], kTileLd, lane);  // + L32 T20
    st16_f32(&sm.scr[3][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(3, 3)][0][0], kTileLd, &sm.scr[3][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(3, 0)][0][0], t2, -1.f, lane);
  }
  __syncthreads();

  // ---- T' = T diag(beta e^G / ||k||), T'' = T diag(beta): fp16 granules of 8
  //      column positions (two token quads each), swizzled ----
  uint16_t* twrec = reinterpret_cast<uint16_t*>(rec + Rec::TW);
  uint16_t* tbrec = reinterpret_cast<uint16_t*>(rec + Rec::TB);
  for (int e = tid; e < 2 * kC * 8; e += NT) {
    const int which = e >> 9;  // 0: T', 1: T''
    const int t = (e >> 3) & 63, gp = e & 7;
    if ((gp >> 2) > (t >> 5)) continue;  // above the diagonal blocks: not stored
    const float* c = which ? sm.bt : sm.cw;
    const float4 a = t_quad(sm.Tp, c, t, quad_of_pos(2 * gp));
    const float4 b = t_quad(sm.Tp, c, t, quad_of_pos(2 * gp + 1));
    uint4 pk;
    pk.x = f2h2(a.x, a.y);
    pk.y = f2h2(a.z, a.w);
    pk.z = f2h2(b.x, b.y);
    pk.w = f2h2(b.z, b.w);
    *reinterpret_cast<uint4*>(&(which ? tbrec : twrec)[tri_off(t, 8 * gp)]) = pk;
  }
}

// ============================================================ state kernel ==
template <int D>
struct __align__(16) StateStage {
  uint16_t Q[kC * D];     // raw q rows (fp16), swz<D>
  uint16_t Kt[D * kC];    // k^ transposed: row = key, token positions, swz<64>
  uint16_t Vt[kCB * kC];  // v transposed: row = value column, token positions, swz<64>
  uint16_t W[kC * D];     // W = T diag(beta e^G) K^ rows (fp16), swz<D>
  uint16_t Tb[3 * 1024];  // record TB
  uint16_t A[3 * 1024];   // record AQ
  float vec[256];         // record VEC: cQ[64], cK[64], e^gamma
};

template <int D>
struct __align__(16) StateSmem {
  StateStage<D> st[2];
  uint16_t out[2][kC * kCB];  // bf16 output tiles of the last two chunks, swz<64>
};

constexpr int kChainWaves = 2;  // 32 state columns each
constexpr int kProdWaves = 4;

// Producer roles.  Waves are placed on the SIMDs round-robin, so chain waves
// 0 and 1 share their SIMDs with producer waves 4 and 5, while waves 2 and 3
// have a SIMD each.  Waves 2 and 3 ("K waves", pw = 0, 1) take the MFMA
// work: for their key tiles kt = pw, pw + 2 (D = 128) they transpose the K
// rows into K^T and multiply them by T' into the matching columns of W, so
// everything they read back from LDS they wrote themselves; they also store
// the previous chunk's outputs.  Waves 4 and 5 (pw = 2, 3) stage V^T, the raw
// Q rows and the record blocks the chain reads (13 blocks of 1 KiB: Tb and A
// (12), vec (1)).
constexpr int kRecBlocks = 13;

// Per-lane prefetch registers of one chunk, one struct per role.
template <int D>
struct KPrefetch {                    // K waves
  static constexpr int NKT = D / 64;  // key tiles per K wave
  s16x8_t k[NKT][2][2];               // K rows: key tile pw + 2u, token tile tt, key k-step h
  s16x8_t tw[6];                      // T' fragments (fp16 bits): (nt 0, ks 0..1), (nt 1, ks 0..3)
};

template <int D>
struct VPrefetch {                    // V / Q / record waves
  static constexpr int NQ = D / 16;   // Q granules per lane
  static constexpr int NREC = 7;      // record blocks per wave (ceil(13 / 2))
  s16x8_t v[2][2];                    // V rows of V^T task 2 (pw - 2) + u, k-step h
  s16x8_t q[NQ];
  s16x8_t rec[NREC];
};

// byte offset in the record of the staged 1 KiB block b (Tb, A, vec)
__device__ __forceinline__ int rec_block_src(int b) { return b < 12 ? Rec::TB + b * 1024 : Rec::VEC; }

// Identity fragment (bf16 B operand) of k-step h of a 32-wide column tile:
// lane (n, g) has a 1 at slot e iff 16 h + 8 g + e == n.
__device__ __forceinline__ s16x8_t ident_frag(int h, int n, int g) {
  s16x8_t f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] = (16 * h + 8 * g + e == n) ? static_cast<short>(0x3f80) : static_cast<short>(0);
  return f;
}

__device__ __forceinline__ f32x16_t mfma32_bf16(const s16x8_t& a, const s16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gdn::bf16x8_t, a),
                                                 __builtin_bit_cast(gdn::bf16x8_t, b), c, 0, 0, 0);
}

// The prefetches issue the global loads of chunk (tok0, len) for this lane.
// The chunk bases are wave-uniform; lane offsets are 32-bit.  Nothing here
// consumes a loaded value, so the loads stay in flight until staging.  Rows
// past the sequence end re-read its last token: those tokens carry zero
// weights in T', T'' and cK, and their outputs are not stored.
template <int D>
__device__ __forceinline__ void k_prefetch(KPrefetch<D>& p, const uint16_t* kh, int sk, const uint8_t* rec,
                                           int64_t tok0, int len, int pw, int lane) {
  const int li = lane & 31, g = lane >> 5;
  const uint16_t* kc = kh + tok0 * sk;
#pragma unroll
  for (int u = 0; u < KPrefetch<D>::NKT; ++u)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int off = min(32 * tt + li, len - 1) * sk + 32 * (pw + 2 * u) + 8 * g;
      p.k[u][tt][0] = *reinterpret_cast<const s16x8_t*>(kc + off);
      p.k[u][tt][1] = *reinterpret_cast<const s16x8_t*>(kc + off + 16);
    }
  const uint16_t* twr = reinterpret_cast<const uint16_t*>(rec + Rec::TW);
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) p.tw[ks] = *reinterpret_cast<const s16x8_t*>(twr + tri_off(li, 16 * ks + 8 * g));
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    p.tw[2 + ks] = *reinterpret_cast<const s16x8_t*>(twr + tri_off(32 + li, 16 * ks + 8 * g));
}

template <int D>
__device__ __forceinline__ void v_prefetch(VPrefetch<D>& p, const uint16_t* qh, int sq, const uint16_t* vh, int sv,
                                           const uint8_t* rec, int64_t tok0, int len, int pv, int lane) {
  const int li = lane & 31, g = lane >> 5;
  const uint16_t* vc = vh + tok0 * sv;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int task = 2 * pv + u;
    const int tt = task & 1, vt = task >> 1;
    const int off = min(32 * tt + li, len - 1) * sv + 32 * vt + 8 * g;
    p.v[u][0] = *reinterpret_cast<const s16x8_t*>(vc + off);
    p.v[u][1] = *reinterpret_cast<const s16x8_t*>(vc + off + 16);
  }
  const uint16_t* qc = qh + tok0 * sq;
  const int plane = pv * 64 + lane;
#pragma unroll
  for (int u = 0; u < VPrefetch<D>::NQ; ++u) {
    const int id = plane + 128 * u;
    const int t = id / (D / 8), c8 = id % (D / 8);
    p.q[u] = *reinterpret_cast<const s16x8_t*>(qc + min(t, len - 1) * sq + 8 * c8);
  }
#pragma unroll
  for (int u = 0; u < VPrefetch<D>::NREC; ++u) {
    const int b = min(pv + 2 * u, kRecBlocks - 1);  // past the end: a repeat, not staged
    p.rec[u] = *reinterpret_cast<const s16x8_t*>(rec + rec_block_src(b) + 16 * lane);
  }
}

// raw bf16 -> fp16 (exact within the fp16 range)
__device__ __forceinline__ h16x8_t bf8_to_h8_raw(const s16x8_t& x) {
  const u32x4_t u = __builtin_bit_cast(u32x4_t, x);
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = f2h2(lo_half(u[p]), hi_half(u[p]));
  return __builtin_bit_cast(h16x8_t, r);
}

// K waves: K^T of their key tiles by bf16 identity products (C = K I of a
// 32-token tile gives lane (key n, g) the tokens 8i + 4g + r, which belong at
// positions 8g + 0..7 and 16 + 8g + 0..7; exact), then W = T' K as
// W^T = K^T T'^T: the A operand reads the K^T rows this wave just wrote, in
// qswap order, so lane (token t, g) ends up with keys 32 kt + 8 g + 0..7 and
// 32 kt + 16 + 8 g + 0..7, two plain 16-byte pieces of row t of W.  k stays
// unnormalised (1/||k|| is folded into T' and cK).
template <int D>
__device__ __forceinline__ void k_stage(const KPrefetch<D>& p, StateStage<D>& S, int pw, int lane,
                                        const s16x8_t& id0, const s16x8_t& id1) {
  const int li = lane & 31, g = lane >> 5;
#pragma unroll
  for (int u = 0; u < KPrefetch<D>::NKT; ++u) {
    const int kt = pw + 2 * u;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x16_t c = zero16();
      c = mfma32_bf16(p.k[u][tt][0], id0, c);
      c = mfma32_bf16(p.k[u][tt][1], id1, c);
      const int row = 32 * kt + li;
      *reinterpret_cast<h16x8_t*>(&S.Kt[swz<kC>(row, 32 * tt + 8 * g)]) = pack_h8<0>(c);
      *reinterpret_cast<h16x8_t*>(&S.Kt[swz<kC>(row, 32 * tt + 16 + 8 * g)]) = pack_h8<8>(c);
    }
  }
  wave_sync();  // the K^T rows are read back by this wave only
  h16x8_t tw[6];
#pragma unroll
  for (int j = 0; j < 6; ++j) tw[j] = __builtin_bit_cast(h16x8_t, p.tw[j]);
#pragma unroll
  for (int u = 0; u < KPrefetch<D>::NKT; ++u) {
    const int kt = pw + 2 * u;
    const int arow = qswap(32 * kt + li);
    h16x8_t kf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kf[ks] = ld_h8(S.Kt, swz<kC>(arow, 16 * ks + 8 * g));
    f32x16_t c0 = zero16(), c1 = zero16();
    c0 = mfma32(kf[0], tw[0], c0);
    c1 = mfma32(kf[0], tw[2], c1);
    c0 = mfma32(kf[1], tw[1], c0);
    c1 = mfma32(kf[1], tw[3], c1);
    c1 = mfma32(kf[2], tw[4], c1);
    c1 = mfma32(kf[3], tw[5], c1);
    *reinterpret_cast<h16x8_t*>(&S.W[swz<D>(li, 32 * kt + 8 * g)]) = pack_h8<0>(c0);
    *reinterpret_cast<h16x8_t*>(&S.W[swz<D>(li, 32 * kt + 16 + 8 * g)]) = pack_h8<8>(c0);
    *reinterpret_cast<h16x8_t*>(&S.W[swz<D>(32 + li, 32 * kt + 8 * g)]) = pack_h8<0>(c1);
    *reinterpret_cast<h16x8_t*>(&S.W[swz<D>(32 + li, 32 * kt + 16 + 8 * g)]) = pack_h8<8>(c1);
  }
}

// V / Q / record waves: record blocks (Tb, A, vec), V^T by identity
// products, raw q rows as fp16 (1/||q|| is folded into cQ).
template <int D>
__device__ __forceinline__ void v_stage(const VPrefetch<D>& p, StateStage<D>& S, int pv, int lane,
                                        const s16x8_t& id0, const s16x8_t& id1) {
  const int li = lane & 31, g = lane >> 5;
#pragma unroll
  for (int u = 0; u < VPrefetch<D>::NREC; ++u) {
    const int b = pv + 2 * u;
    if (b < kRecBlocks) {
      uint8_t* dst = b < 12 ? reinterpret_cast<uint8_t*>(S.Tb) + b * 1024 : reinterpret_cast<uint8_t*>(S.vec);
      *reinterpret_cast<s16x8_t*>(dst + 16 * lane) = p.rec[u];
    }
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int task = 2 * pv + u;
    const int tt = task & 1, vt = task >> 1;
    f32x16_t c = zero16();
    c = mfma32_bf16(p.v[u][0], id0, c);
    c = mfma32_bf16(p.v[u][1], id1, c);
    const int row = 32 * vt + li;
    *reinterpret_cast<h16x8_t*>(&S.Vt[swz<kC>(row, 32 * tt + 8 * g)]) = pack_h8<0>(c);
    *reinterpret_cast<h16x8_t*>(&S.Vt[swz<kC>(row, 32 * tt + 16 + 8 * g)]) = pack_h8<8>(c);
  }
  const int plane = pv * 64 + lane;
#pragma unroll
  for (int u = 0; u < VPrefetch<D>::NQ; ++u) {
    const int id = plane + 128 * u;
    const int t = id / (D / 8), c8 = id % (D / 8);
    *reinterpret_cast<h16x8_t*>(&S.Q[swz<D>(t, 8 * c8)]) = bf8_to_h8_raw(p.q[u]);
  }
}

// K waves: store one chunk's output tile (bf16 [64 tokens][64 columns] in
// LDS, swz<64>) to o with 16-byte stores, 8 lanes per token row.
template <int D>
__device__ __forceinline__ void store_out(const uint16_t* out, uint16_t* o, int64_t tok0, int len, int Hv, int h,
                                          int cb, int pw, int lane) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int id = pw * 64 + lane + 128 * u;
    const int row = id >> 3, gr = id & 7;
    if (row < len)
      *reinterpret_cast<uint4*>(o + ((tok0 + row) * Hv + h) * D + cb * kCB + 8 * gr) =
          *reinterpret_cast<const uint4*>(out + swz<kCB>(row, 8 * gr));
  }
}

// grid = 8 * ceil(n_seqs * Hv * NCB / 8), NCB = D / 64; block = 64 * 6.
// Workgroup (sequence r, value head h, column block cb): waves 0, 1 own the
// state columns cb*64 + 32 w .. + 32 (the chain); waves 2..5 stage chunks
// and store outputs.  One workgroup barrier per chunk: the producer fills the
// stage buffer the chain is not reading and stores the output tile the chain
// wrote in the previous chunk; no producer wave reads what another one wrote.
template <int D>
__global__ __launch_bounds__(64 * (kChainWaves + kProdWaves)) void chunk_state_kernel(
    const uint16_t* __restrict__ q, int64_t sq, const uint16_t* __restrict__ k, int64_t sk,
    const uint16_t* __restrict__ v, int64_t sv, const uint8_t* __restrict__ ws, const float* h0, float* hT,
    const int64_t* __restrict__ ids, int64_t sstride, const int64_t* __restrict__ cu, int n_seqs, int Hk,
    int Hv, uint16_t* __restrict__ o) {
  constexpr int NCB = D / kCB;
  constexpr int NR = D / 32;  // 32-row tiles of the state
  constexpr int KS = D / 16;  // k-steps over keys
  __shared__ StateSmem<D> sm;
  __shared__ long long s_base;

  const int64_t wi = gdn::xcd_remap(blockIdx.x, static_cast<int64_t>(n_seqs) * Hv * NCB);
  if (wi < 0) return;
  const int cb = static_cast<int>(wi % NCB);
  const int h = static_cast<int>((wi / NCB) % Hv);
  const int r = static_cast<int>(wi / (static_cast<int64_t>(NCB) * Hv));
  const int64_t bos = cu[r];
  const int64_t seqlen = cu[r + 1] - bos;
  const int64_t nch = chunks_of(seqlen);
  const int kh = h / (Hv / Hk);

  // first workspace chunk of this sequence: sum of earlier sequences' chunks
  if (threadIdx.x < 64) {
    long long part = 0;
    for (int rr = threadIdx.x; rr < r; rr += 64) part += chunks_of(cu[rr + 1] - cu[rr]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
    if (threadIdx.x == 0) s_base = part;
  }
  __syncthreads();
  const int64_t cbase = s_base;
  const uint8_t* rec0 = ws + (cbase * Hv + h) * Rec::BYTES;
  const int64_t rec_stride = static_cast<int64_t>(Hv) * Rec::BYTES;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, g = lane >> 5;

  if (wave >= kChainWaves) {
    // ---------------------------------------------------------- producer --
    const int pw = wave - kChainWaves;
    const uint16_t* qh = q + static_cast<int64_t>(kh) * D;
    const uint16_t* khp = k + static_cast<int64_t>(kh) * D;
    const uint16_t* vh = v + static_cast<int64_t>(h) * D + cb * kCB;
    if (nch == 0) return;
    const int sqi = static_cast<int>(sq), ski = static_cast<int>(sk), svi = static_cast<int>(sv);
    const s16x8_t id0 = ident_frag(0, li, g), id1 = ident_frag(1, li, g);
    // The prefetch of chunk j + 2 is issued as soon as chunk j + 1 has left
    // the registers, so its loads have a whole chunk of chain work to land.
#define GDN_LEN(j_) static_cast<int>(min<int64_t>(kC, seqlen - (j_) * kC))
    if (pw < 2) {
      KPrefetch<D> p;
      k_prefetch<D>(p, khp, ski, rec0, bos, GDN_LEN(0), pw, lane);
      k_stage<D>(p, sm.st[0], pw, lane, id0, id1);
      if (nch > 1) k_prefetch<D>(p, khp, ski, rec0 + rec_stride, bos + kC, GDN_LEN(1), pw, lane);
      gdn::lds_barrier();
      for (int64_t j = 0; j < nch; ++j) {
        if (j + 1 < nch) {
          k_stage<D>(p, sm.st[(j + 1) & 1], pw, lane, id0, id1);
          if (j + 2 < nch)
            k_prefetch<D>(p, khp, ski, rec0 + (j + 2) * rec_stride, bos + (j + 2) * kC, GDN_LEN(j + 2), pw, lane);
        }
        if (j > 0) store_out<D>(sm.out[(j - 1) & 1], o, bos + (j - 1) * kC, kC, Hv, h, cb, pw, lane);
        gdn::lds_barrier();
      }
      store_out<D>(sm.out[(nch - 1) & 1], o, bos + (nch - 1) * kC, GDN_LEN(nch - 1), Hv, h, cb, pw, lane);
    } else {
      const int pv = pw - 2;
      VPrefetch<D> p;
      v_prefetch<D>(p, qh, sqi, vh, svi, rec0, bos, GDN_LEN(0), pv, lane);
      v_stage<D>(p, sm.st[0], pv, lane, id0, id1);
      if (nch > 1) v_prefetch<D>(p, qh, sqi, vh, svi, rec0 + rec_stride, bos + kC, GDN_LEN(1), pv, lane);
      gdn::lds_barrier();
      for (int64_t j = 0; j < nch; ++j) {
        if (j + 1 < nch) {
          v_stage<D>(p, sm.st[(j + 1) & 1], pv, lane, id0, id1);
          if (j + 2 < nch)
            v_prefetch<D>(p, qh, sqi, vh, svi, rec0 + (j + 2) * rec_stride, bos + (j + 2) * kC, GDN_LEN(j + 2), pv,
                          lane);
        }
        gdn::lds_barrier();
      }
    }
#undef GDN_LEN
    return;
  }

  // -------------------------------------------------------------- chain --
  const int64_t srow = ids ? ids[r] : r;
  const int vc0 = cb * kCB + 32 * wave;  // first state column of this wave
  f32x16_t S[NR];
  if (h0) {
    const float* hp = h0 + srow * sstride + static_cast<int64_t>(h) * D * D + vc0 + li;
#pragma unroll
    for (int rt = 0; rt < NR; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          S[rt][4 * i + rr] = hp[static_cast<int64_t>(qswap(32 * rt + 8 * i + 4 * g + rr)) * D];
  } else {
#pragma unroll
    for (int rt = 0; rt < NR; ++rt) S[rt] = zero16();
  }
  if (nch > 0) gdn::lds_barrier();
  for (int64_t jc = 0; jc < nch; ++jc) {
    const StateStage<D>& B = sm.st[jc & 1];
    // Re-derive lane indices from an opaque copy each chunk so the compiler
    // does not keep every lane-dependent address live across the loop.
    int tid_l = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid_l));
    const int ln = tid_l & 63;
    const int m = ln & 31, lgp = ln >> 5;

    // Operand fragments of each product are read from LDS as one batch ahead
    // of its MFMAs, so the reads overlap each other instead of each MFMA
    // waiting out an LDS latency.
    // U = T'' V (rows = tokens, cols = this wave's 32 value columns)
    f32x16_t U[2];
    {
      h16x8_t vf[4], tf[6];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) vf[ks] = ld_h8(B.Vt, swz<kC>(32 * wave + m, 16 * ks + 8 * lgp));
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) tf[ks] = ld_h8(B.Tb, tri_off(m, 16 * ks + 8 * lgp));
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) tf[2 + ks] = ld_h8(B.Tb, tri_off(32 + m, 16 * ks + 8 * lgp));
      __builtin_amdgcn_sched_barrier(0);  // keep the batch of reads ahead of the products
      U[0] = mfma32(tf[0], vf[0], zero16());
      U[1] = mfma32(tf[2], vf[0], zero16());
      U[0] = mfma32(tf[1], vf[1], U[0]);
      U[1] = mfma32(tf[3], vf[1], U[1]);
      U[1] = mfma32(tf[4], vf[2], U[1]);
      U[1] = mfma32(tf[5], vf[3], U[1]);
    }
    // S as fp16 fragments (B operand of W S, A operand of S^T Q^T)
    h16x8_t Sh[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) Sh[s] = (s & 1) ? pack_h8<8>(S[s >> 1]) : pack_h8<0>(S[s >> 1]);
    // Vn = U - W S, both 32-token tiles interleaved
    {
      h16x8_t wf[2][KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        wf[0][s] = ld_h8(B.W, swz<D>(m, 16 * s + 8 * lgp));
        wf[1][s] = ld_h8(B.W, swz<D>(32 + m, 16 * s + 8 * lgp));
      }
      __builtin_amdgcn_sched_barrier(0);
      f32x16_t a0 = zero16(), a1 = zero16();
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        a0 = mfma32(wf[0][s], Sh[s], a0);
        a1 = mfma32(wf[1][s], Sh[s], a1);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        U[0][e] -= a0[e];
        U[1][e] -= a1[e];
      }
    }
    // Vn (for A Vn) and Vn' = diag(cK) Vn (for the state update) as fp16
    h16x8_t Vh[4], Vk[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) Vh[s] = (s & 1) ? pack_h8<8>(U[s >> 1]) : pack_h8<0>(U[s >> 1]);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4_t ck = *reinterpret_cast<const f32x4_t*>(&B.vec[kC + 32 * mt + 8 * i + 4 * lgp]);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) U[mt][4 * i + rr] *= ck[rr];
      }
#pragma unroll
    for (int s = 0; s < 4; ++s) Vk[s] = (s & 1) ? pack_h8<8>(U[s >> 1]) : pack_h8<0>(U[s >> 1]);
    // S <- e^gamma S + K^T Vn'  (the old S lives on in Sh for the outputs)
    {
      h16x8_t kf[NR][4];
#pragma unroll
      for (int rt = 0; rt < NR; ++rt)
#pragma unroll
        for (int s = 0; s < 4; ++s) kf[rt][s] = ld_h8(B.Kt, swz<kC>(qswap(32 * rt + m), 16 * s + 8 * lgp));
      const float eg = B.vec[2 * kC];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int rt = 0; rt < NR; ++rt)
#pragma unroll
        for (int e = 0; e < 16; ++e) S[rt][e] *= eg;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int rt = 0; rt < NR; ++rt) S[rt] = mfma32(kf[rt][s], Vk[s], S[rt]);
    }
    // O^T = diag(cQ) S^T Q^T + Vn^T A^T, per 32-token tile; the k-steps of
    // S^T Q^T alternate between two accumulators so the MFMAs do not wait on
    // each other's results
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      h16x8_t qf[KS], af[4];
#pragma unroll
      for (int s = 0; s < KS; ++s) qf[s] = ld_h8(B.Q, swz<D>(32 * nt + m, 16 * s + 8 * lgp));
#pragma unroll
      for (int s = 0; s < 2 * nt + 2; ++s) af[s] = ld_h8(B.A, tri_off(32 * nt + m, 16 * s + 8 * lgp));
      const float cq = B.vec[32 * nt + m];
      __builtin_amdgcn_sched_barrier(0);
      f32x16_t acc = zero16(), acc1 = zero16();
#pragma unroll
      for (int s = 0; s < KS; s += 2) {
        acc = mfma32(Sh[s], qf[s], acc);
        acc1 = mfma32(Sh[s + 1], qf[s + 1], acc1);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = (acc[e] + acc1[e]) * cq;
#pragma unroll
      for (int s = 0; s < 2 * nt + 2; ++s) acc = mfma32(Vh[s], af[s], acc);
      // lane (token t, g) holds value columns 8 i + 4 g + 0..3 of its 32;
      // the producer's K waves store the tile after the chunk barrier
      uint16_t* ob = sm.out[jc & 1];
      const int t = 32 * nt + m;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint2 pk;
        pk.x = gdn::f2bf2(acc[4 * i], acc[4 * i + 1]);
        pk.y = gdn::f2bf2(acc[4 * i + 2], acc[4 * i + 3]);
        *reinterpret_cast<uint2*>(&ob[swz<kCB>(t, 32 * wave + 8 * i + 4 * lgp)]) = pk;
      }
    }
    gdn::lds_barrier();
  }

  if (hT) {
    float* hp = hT + srow * sstride + static_cast<int64_t>(h) * D * D + vc0 + li;
#pragma unroll
    for (int rt = 0; rt < NR; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          hp[static_cast<int64_t>(qswap(32 * rt + 8 * i + 4 * g + rr)) * D] = S[rt][4 * i + rr];
  }
}

template <int D>
int launch_chunk(const uint16_t* q, int64_t sq, const uint16_t* k, int64_t sk, const uint16_t* v,
                 int64_t sv, const float* g, const uint16_t* beta, const float* h0, float* hT,
                 const int64_t* ids, int64_t sstride, const int64_t* cu, int n_seqs, int64_t nc_bound,
                 int Hk, int Hv, float scale, int l2norm, uint16_t* o, uint8_t* ws, hipStream_t stream) {
  const int64_t lwork = nc_bound * Hv;
  const int64_t lgrid = gdn::kNumXcd * ((lwork + gdn::kNumXcd - 1) / gdn::kNumXcd);
  chunk_prep_kernel<D><<<dim3(static_cast<unsigned>(lgrid)), dim3(256), 0, stream>>>(
      q, sq, k, sk, g, beta, cu, n_seqs, nc_bound, Hk, Hv, scale, l2norm, ws);
  const int st = gdn_launch_status();
  if (st != GDN_OK) return st;
  const int64_t cwork = static_cast<int64_t>(n_seqs) * Hv * (D / kCB);
  const int64_t cgrid = gdn::kNumXcd * ((cwork + gdn::kNumXcd - 1) / gdn::kNumXcd);
  chunk_state_kernel<D><<<dim3(static_cast<unsigned>(cgrid)), dim3(64 * (kChainWaves + kProdWaves)), 0, stream>>>(
      q, sq, k, sk, v, sv, ws, h0, hT, ids, sstride, cu, n_seqs, Hk, Hv, o);
  return gdn_launch_status();
}

}  // namespace

extern "C" int64_t gdn_chunk_prefill_workspace_size(int64_t N, int n_seqs, int Hv, int D) {
  if (N < 0 || n_seqs < 0 || Hv <= 0 || (D != 64 && D != 128)) return -1;
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  return nc_bound * Hv * Rec::BYTES;
}

extern "C" int gdn_chunk_prefill(const uint16_t* q, int64_t sq_tok, const uint16_t* k,
                                 int64_t sk_tok, const uint16_t* v, int64_t sv_tok, const float* g,
                                 const uint16_t* beta, const float* h0, float* hT,
                                 const int64_t* state_ids, int64_t state_stride,
                                 const int64_t* cu_seqlens, int n_seqs, int64_t N, int Hk, int Hv,
                                 int D, float scale, int l2norm, uint16_t* o, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (n_seqs < 0 || N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return GDN_ERR_INVALID_ARG;
  if (n_seqs == 0) return GDN_OK;
  if (!q || !k || !v || !g || !beta || !cu_seqlens || !o || !workspace) return GDN_ERR_INVALID_ARG;
  // 16-byte row fragments of q / k / v, 8-byte output pieces, 256-byte workspace records
  // token strides: multiples of 8 elements; the state kernel addresses a
  // chunk's rows with 32-bit offsets (64 * stride < 2^31)
  if (sq_tok % 8 || sk_tok % 8 || sv_tok % 8 || reinterpret_cast<uintptr_t>(q) % 16 ||
      sq_tok >= (1LL << 24) || sk_tok >= (1LL << 24) || sv_tok >= (1LL << 24) ||
      reinterpret_cast<uintptr_t>(k) % 16 || reinterpret_cast<uintptr_t>(v) % 16 ||
      reinterpret_cast<uintptr_t>(o) % 8 ||
      reinterpret_cast<uintptr_t>(workspace) % 256 ||
      ((h0 || hT) && state_stride < static_cast<int64_t>(Hv) * D * D))
    return GDN_ERR_INVALID_ARG;
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  if (workspace_bytes < nc_bound * Hv * Rec::BYTES) return GDN_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  if (D == 128)
    return launch_chunk<128>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids, state_stride,
                             cu_seqlens, n_seqs, nc_bound, Hk, Hv, scale, l2norm, o, ws, s);
  return launch_chunk<64>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids, state_stride,
                          cu_seqlens, n_seqs, nc_bound, Hk, Hv, scale, l2norm, o, ws, s);
}
