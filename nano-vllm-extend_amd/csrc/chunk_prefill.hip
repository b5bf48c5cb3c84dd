// Chunked gated delta rule over packed varlen sequences, chunk size 64.
//
// Per chunk (rows t, s in [0, 64); G = inclusive cumsum of g in the chunk,
// gamma = G[63]; k^, q^ = L2-normalised rows; the algorithm of the torch
// port at nanovllm/models/qwen3_5.py:152-227):
//   L    = strict_lower( beta_t k^_t.k^_s e^{G_t-G_s} )
//   T    = (I + L)^-1                       (the reference's forward substitution)
//   W    = T diag(beta e^G) K^,   U = T diag(beta) V
//   Vn   = U - W S
//   O    = diag(e^G) Q^ S + lower_incl( q^_t.k^_s e^{G_t-G_s} ) Vn
//   S   <- e^gamma S + K^T diag(e^{gamma-G}) Vn
//
// Two kernels.  Everything that does not depend on the recurrent state S
// (K K^T, Q K^T, the triangular inverse, W, U) is independent across
// chunks, so chunk_local_kernel computes it for every (chunk, value head)
// in parallel and writes one record per chunk-head into a workspace.
// chunk_chain_kernel then walks each (sequence, value head) chunk by chunk
// with its slice of S in registers; only the S-dependent products are left
// on that sequential path.
//
// Numerics.  q, k, v arrive in bf16, which is exact as an MFMA operand, and
// the L2 norm is a per-row scale; so K K^T, Q K^T, W = T' K_raw and the K
// side of K^T Vn use the raw bf16 rows and apply the scales in fp32.  The
// remaining fp32 operands are split into hi + lo bf16 terms: T'' (U), S (in
// W S and Q S), Vn (K^T Vn) and both sides of A_qk Vn (three passes).  The
// triangular inverse stays in fp32 (fp32 MFMA, blocked 16x16).
//
// Layout trick.  The MFMA C fragment of two vertically adjacent 16x16 tiles
// holds, per lane group, exactly the 8 contraction values a B fragment
// needs, under a fixed permutation of the contraction index.  Applying the
// same permutation to the A side lets S and Vn feed the next products
// straight from registers: the state chain of a wave never touches LDS and
// needs no cross-wave synchronisation (state columns are independent).
#include "gdn_common.h"

namespace {

using gdn::f32x4_t;
using gdn::s16x4_t;
using gdn::s16x8_t;

constexpr int kC = 64;  // chunk size

// ---- workspace record of one (chunk, value head) ----
// A sequence of 1 KiB blocks.  Each bf16 block is one MFMA A operand of the
// chain kernel in lane order (lane l's 8 values at bytes [16 l, 16 l + 16)),
// already in the permuted contraction order of perm_frag; so the chain stages
// a record with linear 16-byte copies and reads every operand with one
// conflict-free 16-byte LDS read per lane.
//   W   [mt][kt]   rows 16 mt.. of W = T' K_raw, key dims 32 kt..
//   Q   [mt][kt]   raw bf16 q rows (zero past the sequence end)
//   K   [mt][kt]   key dims 16 mt.. of K_raw^T, tokens 32 kt..
//   AH, AL         the six (mt, kt) blocks of lower(A_qk) with 32 kt <= 16 mt + 15
//   VEC            fp32 cQ[64], cK[64], e^gamma
//   U   [nt][mt]   fp32 C fragments of U = T'' V (value columns 16 nt..)
// Blocks [0, SHARED) are what every wave of a chain workgroup reads; U is
// per wave.
template <int D>
struct Rec {
  static constexpr int KTD = D / 32;
  static constexpr int MTD = D / 16;
  static constexpr int W = 0;
  static constexpr int Q = W + 4 * KTD;
  static constexpr int K = Q + 4 * KTD;
  static constexpr int AH = K + 2 * MTD;
  static constexpr int AL = AH + 6;
  static constexpr int VEC = AL + 6;
  static constexpr int SHARED = VEC + 1;
  static constexpr int U = SHARED;
  static constexpr int BLOCKS = U + 4 * MTD;
  static constexpr int64_t BYTES = static_cast<int64_t>(BLOCKS) * 1024;
};

// block of lower(A_qk) tile (mt, kt), 32 kt <= 16 mt + 15
__device__ __forceinline__ int a_block(int mt, int kt) { return mt < 2 ? mt : 2 * mt - 2 + kt; }

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ s16x8_t zero8() { return s16x8_t{0, 0, 0, 0, 0, 0, 0, 0}; }

__device__ __forceinline__ s16x8_t cat44(s16x4_t a, s16x4_t b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// A fragment with the permuted contraction order: elements 0..3 are
// row[4*lg .. 4*lg+3], elements 4..7 are row[16 + 4*lg .. 16 + 4*lg+3].
__device__ __forceinline__ s16x8_t perm_frag(const uint16_t* row32, int lg) {
  const s16x4_t a = *reinterpret_cast<const s16x4_t*>(row32 + 4 * lg);
  const s16x4_t b = *reinterpret_cast<const s16x4_t*>(row32 + 16 + 4 * lg);
  return cat44(a, b);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lo_half(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float hi_half(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// hi/lo B fragments from the C fragments of tiles (2j, 2j+1).
__device__ __forceinline__ void split_frag(const f32x4_t& t0, const f32x4_t& t1, s16x8_t& fh, s16x8_t& fl) {
  u32x4_t h, l;
  h[0] = gdn::f2bf2(t0[0], t0[1]);
  h[1] = gdn::f2bf2(t0[2], t0[3]);
  h[2] = gdn::f2bf2(t1[0], t1[1]);
  h[3] = gdn::f2bf2(t1[2], t1[3]);
  l[0] = gdn::f2bf2(t0[0] - lo_half(h[0]), t0[1] - hi_half(h[0]));
  l[1] = gdn::f2bf2(t0[2] - lo_half(h[1]), t0[3] - hi_half(h[1]));
  l[2] = gdn::f2bf2(t1[0] - lo_half(h[2]), t1[1] - hi_half(h[2]));
  l[3] = gdn::f2bf2(t1[2] - lo_half(h[3]), t1[3] - hi_half(h[3]));
  fh = __builtin_bit_cast(s16x8_t, h);
  fl = __builtin_bit_cast(s16x8_t, l);
}

// acc += A(16x16) B(16x16), fp32 operands in LDS, fp32 matrix cores.
__device__ __forceinline__ f32x4_t mm16_f32(f32x4_t acc, const float* A, int lda, const float* B, int ldb, int lane) {
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
    acc = gdn::mfma16x16x4f32(A[lr * lda + 4 * kk + lg], B[(4 * kk + lg) * ldb + lr], acc);
  return acc;
}

__device__ __forceinline__ void st16_f32(float* Cp, int ldc, const f32x4_t& acc, float alpha, int lane) {
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) Cp[(4 * lg + i) * ldc + lr] = alpha * acc[i];
}

__device__ __forceinline__ f32x4_t ld16_f32(const float* Cp, int ldc, int lane) {
  const int lr = lane & 15, lg = lane >> 4;
  f32x4_t r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = Cp[(4 * lg + i) * ldc + lr];
  return r;
}

// lower-triangular 16x16 tile index j in [0, 10) -> (mt, nt), mt >= nt
__device__ __forceinline__ void tri_tile(int j, int& mt, int& nt) {
  mt = j >= 6 ? 3 : (j >= 3 ? 2 : (j >= 1 ? 1 : 0));
  nt = j - (mt * (mt + 1)) / 2;
}

__device__ __forceinline__ int64_t chunks_of(int64_t len) { return (len + kC - 1) / kC; }

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

// ============================================================ local kernel ==
// Lower 16x16 tile (mt, nt), nt <= mt, of a 64x64 lower-triangular matrix
// stored as 10 packed tiles; index inverse of tri_tile.
__device__ __forceinline__ int tix(int mt, int nt) { return (mt * (mt + 1)) / 2 + nt; }

constexpr int kTileLd = 20;  // row stride (floats) of a packed fp32 tile

template <int D, int NW>
struct __align__(16) LocalSmem {
  uint16_t Kt[D][kC + 8];  // K^T of the chunk (raw bf16), row = key dim
  union {
    uint16_t Kr[kC][D + 8];  // K row-major (raw bf16): K K^T, K Q^T
    uint16_t Vt[D][kC + 8];  // then V^T (raw bf16): U = T'' V
  } kv;
  float Lp[10][16][kTileLd];  // lower tiles of L (fp32)
  float Tp[10][16][kTileLd];  // lower tiles of T = (I + L)^-1 (fp32)
  float scr[4][16][kTileLd];  // per-wave 16x16 scratch of the solve
  float G[kC], bt[kC], rk[kC], rq[kC];
  float cW[kC], cQ[kC], cK[kC];
  float ssk[kC], ssq[kC];
  float eg_last;
};

// B fragment of X^T for X = T diag(c) (rows t = 16 mt + lr, contraction over
// tokens s = 32 kc + 8 lg + j): X[t][s] = T[t][s] c[s], zero above the
// diagonal tiles.  Read from the packed T tiles, 8 consecutive floats per lane.
__device__ __forceinline__ void t_row8(const float (*Tp)[16][kTileLd], const float* c, int mt, int kc, int lr,
                                       int lg, float x[8]) {
  const int st = 2 * kc + (lg >> 1);  // s tile
  if (st > mt) {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = 0.f;
    return;
  }
  const float4* row = reinterpret_cast<const float4*>(&Tp[tix(mt, st)][lr][(lg & 1) * 8]);
  const float4* cc = reinterpret_cast<const float4*>(&c[32 * kc + 8 * lg]);
  const float4 r0 = row[0], r1 = row[1], c0 = cc[0], c1 = cc[1];
  x[0] = r0.x * c0.x; x[1] = r0.y * c0.y; x[2] = r0.z * c0.z; x[3] = r0.w * c0.w;
  x[4] = r1.x * c1.x; x[5] = r1.y * c1.y; x[6] = r1.z * c1.z; x[7] = r1.w * c1.w;
}

__device__ __forceinline__ s16x8_t pack8(const float x[8]) {
  u32x4_t h;
  h[0] = gdn::f2bf2(x[0], x[1]);
  h[1] = gdn::f2bf2(x[2], x[3]);
  h[2] = gdn::f2bf2(x[4], x[5]);
  h[3] = gdn::f2bf2(x[6], x[7]);
  return __builtin_bit_cast(s16x8_t, h);
}

__device__ __forceinline__ void split8(const float x[8], s16x8_t& hi, s16x8_t& lo) {
  u32x4_t h, l;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    h[p] = gdn::f2bf2(x[2 * p], x[2 * p + 1]);
    l[p] = gdn::f2bf2(x[2 * p] - lo_half(h[p]), x[2 * p + 1] - hi_half(h[p]));
  }
  hi = __builtin_bit_cast(s16x8_t, h);
  lo = __builtin_bit_cast(s16x8_t, l);
}

// grid = 8 * ceil(nc_bound * Hv / 8); block = 64 * NW.  One workgroup per
// (chunk, value head): computes everything that does not depend on S and
// writes the chunk's record.  Every record block is produced in registers in
// the lane order the chain kernel reads (MFMA C fragments of transposed
// products where needed), so LDS holds only K (both layouts, then V^T) and
// the fp32 L / T tiles.
// Two (D = 128) or three (D = 64) workgroups per CU fit in LDS; the second
// launch bound caps the registers so that as many fit in the register file.
template <int D, int NW>
__global__ __launch_bounds__(64 * NW, D == 128 ? 4 : 3) void chunk_local_kernel(
    const uint16_t* __restrict__ q, int64_t sq, const uint16_t* __restrict__ k, int64_t sk,
    const uint16_t* __restrict__ v, int64_t sv, const float* __restrict__ g,
    const uint16_t* __restrict__ beta, const int64_t* __restrict__ cu, int n_seqs, int64_t nc_bound,
    int Hk, int Hv, float scale, int l2norm, uint8_t* __restrict__ ws) {
  using R = Rec<D>;
  constexpr int NT = 64 * NW;
  constexpr int KTD = R::KTD;
  constexpr int MTD = R::MTD;
  constexpr int SEG = D / 8;               // 16-byte segments per row
  constexpr int NSEG1 = kC * SEG / NT;     // row segments per thread
  static_assert(NW >= 4, "the solve uses four waves");
  static_assert(kC * SEG % NT == 0 && NT % SEG == 0, "segment tiling");
  __shared__ LocalSmem<D, NW> sm;

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
  const uint16_t* vh = v + static_cast<int64_t>(h) * D;
  uint8_t* rec = ws + (cidx * Hv + h) * R::BYTES;
  s16x8_t* blk = reinterpret_cast<s16x8_t*>(rec);  // blk[b * 64 + lane]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- phase 1: K (both layouts), row norms of K and Q, gates; V kept in
  //      registers until K row-major is dead ----
  s16x8_t vseg[NSEG1];
  {
#pragma unroll
    for (int j = 0; j < NSEG1; ++j) {
      const int e = tid + NT * j;
      const int t = e / SEG, c8 = e % SEG;
      const int64_t row = tok0 + min(t, len - 1);
      s16x8_t kv8 = *reinterpret_cast<const s16x8_t*>(kh_ + row * sk + c8 * 8);
      s16x8_t qv8 = *reinterpret_cast<const s16x8_t*>(qh + row * sq + c8 * 8);
      s16x8_t vv8 = *reinterpret_cast<const s16x8_t*>(vh + row * sv + c8 * 8);
      if (t >= len) {
        kv8 = zero8();
        qv8 = zero8();
        vv8 = zero8();
      }
      vseg[j] = vv8;
      *reinterpret_cast<s16x8_t*>(&sm.kv.Kr[t][c8 * 8]) = kv8;
      float ks = 0.f, qs = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t kb = static_cast<uint16_t>(kv8[i]);
        sm.Kt[c8 * 8 + i][t] = kb;
        const float kf = gdn::bf2f(kb), qf = gdn::bf2f(static_cast<uint16_t>(qv8[i]));
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
  }
  // Q record blocks straight from global: block (mt, kt), lane pieces
  // q[16 mt + lr][32 kt + 4 lg ..] and [.. + 16 ..] (zero past the end).
  for (int b = wave; b < 4 * KTD; b += NW) {
    const int mt = b / KTD, kt = b % KTD;
    const int t = 16 * mt + lr;
    const uint16_t* qr = qh + (tok0 + min(t, len - 1)) * sq + 32 * kt;
    s16x8_t f = perm_frag(qr, lg);
    if (t >= len) f = zero8();
    blk[(R::Q + b) * 64 + lane] = f;
  }
  __syncthreads();
  if (tid < kC) {
    const int t = tid;
    const float rk = l2norm ? rsqrtf(sm.ssk[t] + 1e-6f) : 1.0f;
    const float rq = l2norm ? rsqrtf(sm.ssq[t] + 1e-6f) : 1.0f;
    const float Gt = sm.G[t];
    const float Gl = sm.G[kC - 1];
    sm.rk[t] = rk;
    sm.rq[t] = rq;
    sm.cW[t] = sm.bt[t] * rk * expf(Gt);
    sm.cQ[t] = rq * scale * expf(Gt);
    sm.cK[t] = rk * expf(Gl - Gt);
    if (t == 0) sm.eg_last = expf(Gl);
    float* vrec = reinterpret_cast<float*>(rec + R::VEC * 1024);
    vrec[t] = sm.cQ[t];
    vrec[kC + t] = sm.cK[t];
    if (t == 0) vrec[2 * kC] = sm.eg_last;
  }
  // K^T record blocks: key rows 16 mt.., tokens 32 kt.. (permuted order)
  for (int b = wave; b < 2 * MTD; b += NW) {
    const int mt = b >> 1, kt = b & 1;
    blk[(R::K + b) * 64 + lane] = perm_frag(&sm.Kt[16 * mt + lr][32 * kt], lg);
  }
  __syncthreads();

  // ---- phase 2a: K K^T -> L (fp32 lower tiles) ----
  for (int j = wave; j < 10; j += NW) {
    int mt, nt;
    tri_tile(j, mt, nt);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KTD; ++kk) {
      const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.kv.Kr[16 * mt + lr][32 * kk + 8 * lg]);
      const s16x8_t b8 = *reinterpret_cast<const s16x8_t*>(&sm.kv.Kr[16 * nt + lr][32 * kk + 8 * lg]);
      acc = gdn::mfma16x16x32(a8, b8, acc);
    }
    const int s = 16 * nt + lr;
    const float rks = sm.rk[s];
    const float Gs = sm.G[s];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * mt + 4 * lg + i;
      sm.Lp[j][4 * lg + i][lr] = s < t ? acc[i] * sm.bt[t] * sm.rk[t] * rks * expf(sm.G[t] - Gs) : 0.f;
    }
  }
  __syncthreads();

  // ---- phase 2b: wave 0 inverts the diagonal blocks; the other waves form
  //      the A_qk record blocks as C fragments of (K Q^T) tile pairs ----
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
    for (int b = wave - 1; b < 6; b += NW - 1) {
      const int mt = b < 2 ? b : 2 + ((b - 2) >> 1);
      const int kt = b < 2 ? 0 : ((b - 2) & 1);
      const int t = 16 * mt + lr;  // the lane's query token (C column)
      // B operand: q row t, key dims 32 kk + 8 lg .. (raw bf16)
      const uint16_t* qr = qh + (tok0 + min(t, len - 1)) * sq + 8 * lg;
      s16x8_t qb[KTD];
#pragma unroll
      for (int kk = 0; kk < KTD; ++kk) qb[kk] = *reinterpret_cast<const s16x8_t*>(qr + 32 * kk);
      const float qscale = sm.rq[t] * scale;
      const float Gt = sm.G[t];
      float a[8];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ns = 2 * kt + half;  // key-token tile
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        if (ns <= mt) {
#pragma unroll
          for (int kk = 0; kk < KTD; ++kk) {
            const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.kv.Kr[16 * ns + lr][32 * kk + 8 * lg]);
            acc = gdn::mfma16x16x32(a8, qb[kk], acc);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int s = 16 * ns + 4 * lg + i;
          a[4 * half + i] = s <= t ? acc[i] * qscale * sm.rk[s] * expf(Gt - sm.G[s]) : 0.f;
        }
      }
      s16x8_t ahi, alo;
      split8(a, ahi, alo);
      blk[(R::AH + b) * 64 + lane] = ahi;
      blk[(R::AL + b) * 64 + lane] = alo;
    }
  }
  __syncthreads();
  // K row-major is dead: V^T takes its place (read in phase 5, after three
  // more barriers)
#pragma unroll
  for (int j = 0; j < NSEG1; ++j) {
    const int e = tid + NT * j;
    const int t = e / SEG, c8 = e % SEG;
#pragma unroll
    for (int i = 0; i < 8; ++i) sm.kv.Vt[c8 * 8 + i][t] = static_cast<uint16_t>(vseg[j][i]);
  }
  // first sub-diagonal: T(j+1, j) = -T(j+1,j+1) L(j+1,j) T(j,j)
  if (wave < 3) {
    const int j = wave, i = j + 1;
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(i, j)][0][0], kTileLd, &sm.Tp[tix(j, j)][0][0], kTileLd, lane);
    st16_f32(&sm.scr[wave][0][0], kTileLd, p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(i, i)][0][0], kTileLd, &sm.scr[wave][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(i, j)][0][0], kTileLd, t2, -1.f, lane);
  } else if (wave == 3) {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(3, 0)][0][0], kTileLd, &sm.Tp[tix(0, 0)][0][0], kTileLd, lane);  // L30 T00
    st16_f32(&sm.scr[3][0][0], kTileLd, p, 1.f, lane);
  }
  __syncthreads();
  // second sub-diagonal: T20, T31; partial sum for T30
  if (wave == 0) {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(2, 0)][0][0], kTileLd, &sm.Tp[tix(0, 0)][0][0], kTileLd, lane);  // L20 T00
    p = mm16_f32(p, &sm.Lp[tix(2, 1)][0][0], kTileLd, &sm.Tp[tix(1, 0)][0][0], kTileLd, lane);  // L21 T10
    st16_f32(&sm.scr[0][0][0], kTileLd, p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(2, 2)][0][0], kTileLd, &sm.scr[0][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(2, 0)][0][0], kTileLd, t2, -1.f, lane);
  } else if (wave == 1) {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(3, 1)][0][0], kTileLd, &sm.Tp[tix(1, 1)][0][0], kTileLd, lane);  // L31 T11
    p = mm16_f32(p, &sm.Lp[tix(3, 2)][0][0], kTileLd, &sm.Tp[tix(2, 1)][0][0], kTileLd, lane);  // L32 T21
    st16_f32(&sm.scr[1][0][0], kTileLd, p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(3, 3)][0][0], kTileLd, &sm.scr[1][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(3, 1)][0][0], kTileLd, t2, -1.f, lane);
  } else if (wave == 3) {
    f32x4_t p = ld16_f32(&sm.scr[3][0][0], kTileLd, lane);
    p = mm16_f32(p, &sm.Lp[tix(3, 1)][0][0], kTileLd, &sm.Tp[tix(1, 0)][0][0], kTileLd, lane);  // + L31 T10
    st16_f32(&sm.scr[3][0][0], kTileLd, p, 1.f, lane);
  }
  __syncthreads();
  // third sub-diagonal: T30
  if (wave == 3) {
    f32x4_t p = ld16_f32(&sm.scr[3][0][0], kTileLd, lane);
    p = mm16_f32(p, &sm.Lp[tix(3, 2)][0][0], kTileLd, &sm.Tp[tix(2, 0)][0][0], kTileLd, lane);  // + L32 T20
    st16_f32(&sm.scr[3][0][0], kTileLd, p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, &sm.Tp[tix(3, 3)][0][0], kTileLd, &sm.scr[3][0][0], kTileLd, lane);
    st16_f32(&sm.Tp[tix(3, 0)][0][0], kTileLd, t2, -1.f, lane);
  }
  __syncthreads();

  // ---- phase 5: W blocks as C fragments of W^T = K^T (T diag(cW))^T tile
  //      pairs, U = (T diag(beta)) V as C fragments (T'' split hi/lo) ----
  for (int b = wave; b < 4 * KTD; b += NW) {
    const int mt = b / KTD, kt = b % KTD;
    s16x8_t tb[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      float x[8];
      t_row8(sm.Tp, sm.cW, mt, kc, lr, lg, x);
      tb[kc] = pack8(x);
    }
    float w8[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int nk = 2 * kt + half;  // key tile
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.Kt[16 * nk + lr][32 * kc + 8 * lg]);
        acc = gdn::mfma16x16x32(a8, tb[kc], acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) w8[4 * half + i] = acc[i];
    }
    blk[(R::W + b) * 64 + lane] = pack8(w8);
  }
  {
    f32x4_t* urec = reinterpret_cast<f32x4_t*>(rec + R::U * 1024);
    for (int nt = wave; nt < MTD; nt += NW) {
      s16x8_t vb[2];
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) vb[kc] = *reinterpret_cast<const s16x8_t*>(&sm.kv.Vt[16 * nt + lr][32 * kc + 8 * lg]);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        f32x4_t u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          if (2 * kc > mt) break;  // T'' is zero above the diagonal tiles
          float x[8];
          t_row8(sm.Tp, sm.bt, mt, kc, lr, lg, x);
          s16x8_t ah, al;
          split8(x, ah, al);
          u = gdn::mfma16x16x32(ah, vb[kc], u);
          u = gdn::mfma16x16x32(al, vb[kc], u);
        }
        urec[(nt * 4 + mt) * 64 + lane] = u;
      }
    }
  }
}

// ============================================================ chain kernel ==
// Double-buffered LDS copy of one chunk's record: the shared blocks plus the
// U blocks of the workgroup's NW column tiles.
template <int D, int NW>
struct __align__(16) ChainSmem {
  static constexpr int NB = Rec<D>::SHARED + 4 * NW;  // 1 KiB blocks per chunk
  s16x8_t buf[2][NB][64];
};

constexpr int kChainLoaders = 2;  // loader waves per chain workgroup

// One loader wave's share of a chunk's copy, global -> LDS with no registers:
// shared blocks b = li, li + kChainLoaders, ..., then the U blocks of the
// workgroup's column tiles.  rec already includes the lane's 16-byte offset;
// the hardware writes lane l's 16 bytes at dst block + 16 l.
template <int D, int NW>
__device__ __forceinline__ void copy_record(const uint8_t* rec, s16x8_t (*dst)[64], int li, int cb) {
  using R = Rec<D>;
  for (int b = li; b < R::SHARED; b += kChainLoaders)
    __builtin_amdgcn_global_load_lds(rec + b * 1024, &dst[b][0], 16, 0, 0);
  const uint8_t* urec = rec + static_cast<int64_t>(R::U + 4 * NW * cb) * 1024;
  for (int b = li; b < 4 * NW; b += kChainLoaders)
    __builtin_amdgcn_global_load_lds(urec + b * 1024, &dst[R::SHARED + b][0], 16, 0, 0);
}

// grid = 8 * ceil(n_seqs * Hv * NCB / 8), NCB = D / (16 NW);
// block = 64 (NW + kChainLoaders).
// Workgroup (sequence r, value head h, column block cb).  Waves 0..NW-1
// compute: wave w owns the state columns [16 nt, 16 nt + 16), nt = cb NW + w.
// Value columns of S evolve independently, so the column blocks of one head
// never communicate.  Waves NW.. only move data: they copy chunk j + 1's
// record into the other LDS buffer (global -> LDS, no registers) while the
// compute waves work on chunk j; one barrier per chunk hands the buffers over.
// The compute waves issue no loads at all inside the loop.  Two loader waves
// keep a whole record in flight (a wave can have at most 63 loads
// outstanding).
template <int D, int NW>
__global__ __launch_bounds__(64 * (NW + kChainLoaders)) void chunk_chain_kernel(
    const uint8_t* __restrict__ ws, const float* h0, float* hT, const int64_t* __restrict__ ids,
    int64_t sstride, const int64_t* __restrict__ cu, int n_seqs, int Hv, uint16_t* __restrict__ o) {
  using R = Rec<D>;
  using SM = ChainSmem<D, NW>;
  constexpr int KTD = R::KTD;
  constexpr int MTD = R::MTD;
  constexpr int NCB = MTD / NW;
  static_assert(MTD % NW == 0, "column blocks tile the head");
  __shared__ SM sm;
  __shared__ long long s_base;

  const int64_t wi = gdn::xcd_remap(blockIdx.x, static_cast<int64_t>(n_seqs) * Hv * NCB);
  if (wi < 0) return;
  const int cb = static_cast<int>(wi % NCB);
  const int h = static_cast<int>((wi / NCB) % Hv);
  const int r = static_cast<int>(wi / (static_cast<int64_t>(NCB) * Hv));
  const int64_t bos = cu[r];
  const int64_t seqlen = cu[r + 1] - bos;
  const int64_t nch = chunks_of(seqlen);

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

  const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave_id >= NW) {
    // ---- loader waves: nch + 1 barriers, matching the compute waves ----
    const int lane = threadIdx.x & 63;
    const int li = wave_id - NW;
    const uint8_t* rec0 = ws + (cbase * Hv + h) * R::BYTES + lane * 16;
    if (nch > 0) copy_record<D, NW>(rec0, sm.buf[0], li, cb);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies have landed in LDS
    gdn::lds_barrier();
    for (int64_t j = 0; j < nch; ++j) {
      if (j + 1 < nch) copy_record<D, NW>(rec0 + (j + 1) * Hv * R::BYTES, sm.buf[(j + 1) & 1], li, cb);
      __builtin_amdgcn_s_waitcnt(0);
      gdn::lds_barrier();
    }
    return;
  }

  // ---- compute waves ----
  const int64_t srow = ids ? ids[r] : r;
  const int nt0 = cb * NW + (threadIdx.x >> 6);
  const int vcol0 = 16 * nt0 + (threadIdx.x & 15);
  const int lg0 = (threadIdx.x & 63) >> 4;
  f32x4_t S[MTD];
  if (h0) {
    const float* hp = h0 + srow * sstride + static_cast<int64_t>(h) * D * D + vcol0;
#pragma unroll
    for (int mt = 0; mt < MTD; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[mt][i] = hp[static_cast<int64_t>(16 * mt + 4 * lg0 + i) * D];
  } else {
#pragma unroll
    for (int mt = 0; mt < MTD; ++mt) S[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  gdn::lds_barrier();  // chunk 0 is in buffer 0

  for (int64_t jc = 0; jc < nch; ++jc) {
    const int64_t c0 = jc * kC;
    const int len = static_cast<int>(min<int64_t>(kC, seqlen - c0));
    const int64_t tok0 = bos + c0;
    // Re-derive the lane indices from an opaque copy each chunk: otherwise the
    // compiler hoists every lane-dependent address out of the loop and keeps
    // them all live in VGPRs, which spills.
    int tid_l = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid_l));
    const int lane = tid_l & 63;
    const int lg = lane >> 4;
    const int lr = lane & 15;
    const int w = __builtin_amdgcn_readfirstlane(tid_l >> 6);
    const int nt = cb * NW + w;
    const int vcol4 = 16 * nt + 4 * lg;  // first of the lane's 4 output columns
    const s16x8_t(*blk)[64] = sm.buf[jc & 1];
    f32x4_t U[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) U[mt] = __builtin_bit_cast(f32x4_t, blk[R::SHARED + 4 * w + mt][lane]);
    const float* vec = reinterpret_cast<const float*>(&blk[R::VEC][0]);

    // W S (Vn = U - W S) and, transposed, O^T = S^T Q^T: the fragments of S
    // serve as the B operand of the first and the A operand of the second, the
    // Q blocks as A and B operand respectively.  The transposed output tile
    // gives each lane 4 consecutive value columns of one token.
    f32x4_t wsum[4], ot[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      wsum[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      ot[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int kt = 0; kt < KTD; ++kt) {
      s16x8_t sh, sl;
      split_frag(S[2 * kt], S[2 * kt + 1], sh, sl);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const s16x8_t wa = blk[R::W + mt * KTD + kt][lane];
        const s16x8_t qa = blk[R::Q + mt * KTD + kt][lane];
        wsum[mt] = gdn::mfma16x16x32(wa, sh, wsum[mt]);
        wsum[mt] = gdn::mfma16x16x32(wa, sl, wsum[mt]);
        ot[mt] = gdn::mfma16x16x32(sh, qa, ot[mt]);
        ot[mt] = gdn::mfma16x16x32(sl, qa, ot[mt]);
      }
    }
    // Vn = U - W S;  O^T_inter *= cQ (per token: lane's token 16 mt + lr)
    f32x4_t vn[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const float cq = vec[16 * mt + lr];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        vn[mt][i] = U[mt][i] - wsum[mt][i];
        ot[mt][i] *= cq;
      }
    }
    // Vn (hi/lo) and Vn' = diag(cK) Vn (hi/lo) fragments, contraction over tokens
    s16x8_t vh_[2], vl_[2], ph[2], pl[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      split_frag(vn[2 * kt], vn[2 * kt + 1], vh_[kt], vl_[kt]);
      const f32x4_t ck0 = *reinterpret_cast<const f32x4_t*>(&vec[kC + 32 * kt + 4 * lg]);
      const f32x4_t ck1 = *reinterpret_cast<const f32x4_t*>(&vec[kC + 32 * kt + 16 + 4 * lg]);
      f32x4_t p0, p1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p0[i] = vn[2 * kt][i] * ck0[i];
        p1[i] = vn[2 * kt + 1][i] * ck1[i];
      }
      split_frag(p0, p1, ph[kt], pl[kt]);
    }
    // O^T += Vn^T A_qk^T (lower-triangular A_qk: only blocks with 32 kt <= 16 mt + 15)
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      f32x4_t acc = ot[mt];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        if (32 * kt > 16 * mt + 15) break;
        const s16x8_t ah = blk[R::AH + a_block(mt, kt)][lane];
        const s16x8_t al = blk[R::AL + a_block(mt, kt)][lane];
        acc = gdn::mfma16x16x32(vh_[kt], ah, acc);
        acc = gdn::mfma16x16x32(vl_[kt], ah, acc);
        acc = gdn::mfma16x16x32(vh_[kt], al, acc);
      }
      const int t = 16 * mt + lr;
      if (t < len) {
        uint2 pk;
        pk.x = gdn::f2bf2(acc[0], acc[1]);
        pk.y = gdn::f2bf2(acc[2], acc[3]);
        *reinterpret_cast<uint2*>(&o[((tok0 + t) * Hv + h) * D + vcol4]) = pk;
      }
    }
    // S <- e^gamma S + K^T Vn'
    const float eg = vec[2 * kC];
#pragma unroll
    for (int mt = 0; mt < MTD; ++mt) {
      f32x4_t acc;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = S[mt][i] * eg;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const s16x8_t ka = blk[R::K + mt * 2 + kt][lane];
        acc = gdn::mfma16x16x32(ka, ph[kt], acc);
        acc = gdn::mfma16x16x32(ka, pl[kt], acc);
      }
      S[mt] = acc;
    }
    gdn::lds_barrier();  // done with this buffer; the next chunk is in the other
  }

  if (hT) {
    float* hp = hT + srow * sstride + static_cast<int64_t>(h) * D * D + vcol0;
#pragma unroll
    for (int mt = 0; mt < MTD; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) hp[static_cast<int64_t>(16 * mt + 4 * lg0 + i) * D] = S[mt][i];
  }
}

template <int D, int NWL, int NWC>
int launch_chunk(const uint16_t* q, int64_t sq, const uint16_t* k, int64_t sk, const uint16_t* v,
                 int64_t sv, const float* g, const uint16_t* beta, const float* h0, float* hT,
                 const int64_t* ids, int64_t sstride, const int64_t* cu, int n_seqs, int64_t nc_bound,
                 int Hk, int Hv, float scale, int l2norm, uint16_t* o, uint8_t* ws, hipStream_t stream) {
  const int64_t lwork = nc_bound * Hv;
  const int64_t lgrid = gdn::kNumXcd * ((lwork + gdn::kNumXcd - 1) / gdn::kNumXcd);
  chunk_local_kernel<D, NWL><<<dim3(static_cast<unsigned>(lgrid)), dim3(64 * NWL), 0, stream>>>(
      q, sq, k, sk, v, sv, g, beta, cu, n_seqs, nc_bound, Hk, Hv, scale, l2norm, ws);
  const int st = gdn_launch_status();
  if (st != GDN_OK) return st;
  const int64_t cwork = static_cast<int64_t>(n_seqs) * Hv * (D / 16 / NWC);
  const int64_t cgrid = gdn::kNumXcd * ((cwork + gdn::kNumXcd - 1) / gdn::kNumXcd);
  chunk_chain_kernel<D, NWC><<<dim3(static_cast<unsigned>(cgrid)), dim3(64 * (NWC + kChainLoaders)), 0, stream>>>(
      ws, h0, hT, ids, sstride, cu, n_seqs, Hv, o);
  return gdn_launch_status();
}

int64_t record_bytes(int D) { return D == 128 ? Rec<128>::BYTES : Rec<64>::BYTES; }

}  // namespace

extern "C" int64_t gdn_chunk_prefill_workspace_size(int64_t N, int n_seqs, int Hv, int D) {
  if (N < 0 || n_seqs < 0 || Hv <= 0 || (D != 64 && D != 128)) return -1;
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  return nc_bound * Hv * record_bytes(D);
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
  if (sq_tok % 8 || sk_tok % 8 || sv_tok % 8 || reinterpret_cast<uintptr_t>(q) % 16 ||
      reinterpret_cast<uintptr_t>(k) % 16 || reinterpret_cast<uintptr_t>(v) % 16 ||
      reinterpret_cast<uintptr_t>(o) % 8 ||
      reinterpret_cast<uintptr_t>(workspace) % 256 ||
      ((h0 || hT) && state_stride < static_cast<int64_t>(Hv) * D * D))
    return GDN_ERR_INVALID_ARG;
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  if (workspace_bytes < nc_bound * Hv * record_bytes(D)) return GDN_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  if (D == 128)
    return launch_chunk<128, 8, 4>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids, state_stride,
                                   cu_seqlens, n_seqs, nc_bound, Hk, Hv, scale, l2norm, o, ws, s);
  return launch_chunk<64, 4, 4>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids, state_stride,
                                cu_seqlens, n_seqs, nc_bound, Hk, Hv, scale, l2norm, o, ws, s);
}
