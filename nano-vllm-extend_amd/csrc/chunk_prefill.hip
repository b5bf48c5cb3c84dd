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
//   chunk_prep_kernel: one workgroup per (chunk, key head), all chunks in
//     parallel, writing one record per value head.  Everything that needs only the chunk's own q, k, g, beta:
//     the row norms, K K^T, Q K^T, the triangular inverse T (fp32), and it
//     writes a 51 KiB record: T'' = T diag(beta) with the column scale cT
//     that makes it -T' = -T diag(beta e^G / |k|),
//     A and A's fp16 rounding residual as fp16 tiles, the per-token scales,
//     and the q rows and K^T as fp16 operand fragments.  The fused variant first computes the gates
//     and the conv1d + SiLU of the chunk's q and k channels from the raw rows.
//   chunk_state_kernel: one workgroup per (sequence, value head, block of 64
//     value columns), persistent over the sequence's chunks.  Producer waves
//     stage the next chunk (the record's K^T; -W = -T' K^ by MFMA; U = T'' V,
//     where the fused variant's V is the conv1d + SiLU of the raw v channels,
//     computed by the U waves) into a double-buffered LDS stage while two
//     chain waves run the state-dependent products of the current chunk with
//     their 128 x 32 slice of S in registers.
//
// Numerics.  Every state-path product runs on the fp16 matrix cores
// (v_mfma_f32_32x32x16_f16, fp32 accumulation): fp16 keeps 11 significant
// bits, and a CPU simulation of one pass against an fp64 recurrence gives
// state rel ~2.6e-4 at the slow decays of trained checkpoints (bf16
// single-pass operands give ~2e-3).  The output's intra-chunk product A Vn,
// which dominated the one-pass output error (mean-rel ~3e-4), runs as three
// products Vh A + Vl A + Vh A_lo over the operands' fp16 roundings and
// residuals (~1e-5).  K is L2-normalised (in fp32) before its fp16 conversion, so its
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
#include <algorithm>
#include <mutex>

#include "gdn_common.h"

namespace {

using gdn::f32x4_t;
using gdn::s16x8_t;

typedef _Float16 h16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kC = 64;   // chunk size (tokens)
constexpr int kCB = 64;  // value columns per state workgroup

__host__ __device__ __forceinline__ int64_t chunks_of(int64_t len) { return (len + kC - 1) / kC; }

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

// fp16x2 -> two fp32 (exact)
__device__ __forceinline__ gdn::f32x2_t h22f(uint32_t u) {
  return __builtin_convertvector(__builtin_bit_cast(h16x2_t, u), gdn::f32x2_t);
}

// the rounding residuals of a pair already packed as f2h2(a, b)
__device__ __forceinline__ uint32_t f2h2_lo(float a, float b, uint32_t hi) {
  const gdn::f32x2_t h = h22f(hi);
  return f2h2(a - h[0], b - h[1]);
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

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- record of one (chunk, value head), byte offsets ----
// Every operand tile is stored in matrix-core fragment order: a fragment is
// 64 lanes x 16 bytes (8 fp16), lane = row % 32 + 32 * (8-column half of its
// 16-column k-step), so a wave moves one fragment as one contiguous KiB.
// Token columns are in position order (position p holds token qswap(p)).
//   TB  [6] frags      T'' = T diag(beta), block-lower-triangular 64x64:
//                      fragment j = (row tile 0, k-steps 0..1), (row tile 1,
//                      k-steps 0..3)
//   AQ  [6] frags      A = lower_incl(scale q^.k^ e^{G_t - G_s}), same order
//   AL  [6] frags      the rounding residual of A: fp16(A_fp32 - fp32(AQ)), same
//                      order, so that A_fp32 = AQ + AL to ~22 significant bits
//   VEC fp32 [256]     cQ[64] = scale e^{G_t} / ||q_t||,
//                      cK[64] = e^{gamma - G_t} / ||k_t|| (0 past the sequence end),
//                      e^gamma, and at 192: cT[64] = -e^{G_t} / ||k_t|| (0 past
//                      the sequence end), the column scale that turns T'' into
//                      -T' = -T diag(beta e^G / ||k||) = T'' diag(cT) (the K waves)
//   QP  [2][D/16]      Q' = diag(cQ) q: [token tile][key step]
//   KT  [D/32][4]      K^T, rows in position order (row p holds key qswap(p)):
//                      [key tile][token step]
// (-T' itself is not stored: the record is the state kernel's main HBM read
// and the prep kernel's main write, and 6 KiB less of it is ~5 % less time.)
struct Rec {
  static constexpr int TB = 0;
  static constexpr int AQ = 6144;
  static constexpr int AL = 12288;
  static constexpr int VEC = 18432;
  static constexpr int QP = 19456;
  static constexpr int CT = 3 * kC;  // float offset of cT in VEC
};
__host__ __device__ constexpr int64_t rec_kt(int D) { return Rec::QP + 128LL * D; }
// bytes of one record (a multiple of 256)
__host__ __device__ constexpr int64_t rec_bytes(int D) { return Rec::QP + 256LL * D; }

// byte offset of fragment f, lane l
__device__ __forceinline__ int frag_byte(int f, int l) { return (f * 64 + l) * 16; }

// byte offset of element (row, col) of a block-lower-triangular 64x64 record
// tile (col / 32 <= row / 32)
__device__ __forceinline__ int tri_frag_byte(int row, int col) {
  const int ks = col >> 4;
  const int j = (row >> 5) == 0 ? ks : 2 + ks;
  return frag_byte(j, (row & 31) + 32 * ((col >> 3) & 1)) + 2 * (col & 7);
}

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

// Identity fragment (bf16 B operand) of k-step h of a 32-wide column tile:
// lane (n, g) has a 1 at slot e iff 16 h + 8 g + e == col(n), with col(n) = n
// (natural) or qswap(n) (so output column n receives input column qswap(n)).
__device__ __forceinline__ s16x8_t ident_frag(int h, int coln, int g) {
  // the slot e = coln - 16 h - 8 g, if in [0, 8): bf16 1.0 in half e & 1 of word e >> 1
  const uint32_t e = static_cast<uint32_t>(coln - 16 * h - 8 * g);
  const uint32_t one = e < 8 ? (0x3f80u << (16 * (e & 1))) : 0u;
  u32x4_t w;
#pragma unroll
  for (int k = 0; k < 4; ++k) w[k] = (e >> 1) == static_cast<uint32_t>(k) ? one : 0u;
  return __builtin_bit_cast(s16x8_t, w);
}

__device__ __forceinline__ f32x16_t mfma32_bf16(const s16x8_t& a, const s16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gdn::bf16x8_t, a),
                                                 __builtin_bit_cast(gdn::bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ h16x8_t as_h8(const s16x8_t& x) { return __builtin_bit_cast(h16x8_t, x); }

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

// LDS of the prep kernel: 37 KiB at D = 128, four workgroups per CU.
template <int D>
struct __align__(16) PrepSmem {
  // The bf16 K rows are last read by the A rows (phase 2b); after that
  // barrier the same bytes hold the off-diagonal tiles of T and the solve's
  // per-wave scratch.
  union {
    uint16_t Kr[kC][D + 8];
    struct {
      float To[6][16][kTileLd];   // T tiles (mt, nt < mt) at mt (mt - 1) / 2 + nt
      float scr[4][16][kTileLd];
    } s;
  } u;
  float Lp[10][16][kTileLd];      // lower tiles of L
  float Td[4][16][kTileLd];       // diagonal tiles of T = (I + L)^-1
  float G[kC], bt[kC], rk[kC], rq[kC], ssk[kC], ssq[kC], cq[kC];
};

// 16x16 tile (mt, nt) of T, nt <= mt
template <int D>
__device__ __forceinline__ float* t_tile(PrepSmem<D>& sm, int mt, int nt) {
  return mt == nt ? &sm.Td[mt][0][0] : &sm.u.s.To[(mt * (mt - 1)) / 2 + nt][0][0];
}

// Row t, token quad Q (tokens 4Q..4Q+3) of T, times c[s]: 4 floats.
template <int D>
__device__ __forceinline__ float4 t_quad(PrepSmem<D>& sm, const float* c, int t, int Q) {
  const int mt = t >> 4, st = Q >> 2;
  if (st > mt) return make_float4(0.f, 0.f, 0.f, 0.f);
  const float4 r = *reinterpret_cast<const float4*>(t_tile(sm, mt, st) + (t & 15) * kTileLd + (Q & 3) * 4);
  const float4 cc = *reinterpret_cast<const float4*>(&c[4 * Q]);
  return make_float4(r.x * cc.x, r.y * cc.y, r.z * cc.z, r.w * cc.w);
}

// quad index (4 tokens) of the tokens at positions [4P, 4P + 4)
__device__ __forceinline__ int quad_of_pos(int P) { return qswap(4 * P) >> 2; }

// Inputs of the fused variant (conv1d + SiLU and the gates computed in the
// prep kernel from the layer's raw inputs).
struct ConvIn {
  const uint16_t* x;       // [N, C] raw q | k | v rows, row stride sx; C = 2 key_dim + Hv D
  int64_t sx;
  const uint16_t* cstate;  // conv state pool: row `slot`, channel c, tap j at
  int64_t ss_seq, ss_ch;   //   cstate + slot*ss_seq + c*ss_ch + j (read here only)
  const int64_t* ids;      // pool rows per sequence (NULL: the sequence index)
  const uint8_t* fresh;    // per sequence, nonzero: zero initial states, pools not read (NULL: none)
  const uint16_t* w;       // [C, 4] conv taps
  int key_dim;             // Hk * D
  const uint16_t* a;       // [N, Hv] gate inputs
  const uint16_t* b;
  const void* A_log;       // [Hv], bf16 or fp32 (param_f32)
  const void* dt_bias;
  int param_f32;
};

// Fused variant, phase 1: causal conv (width 4) + SiLU of the chunk's q and k
// rows (the v channels' conv runs in the state kernel).  Each output row needs
// the 3 raw rows before it: inside the chunk and the previous chunk they are
// rows of x, before a sequence's first token they are the conv state's taps.
// Waves 0-1 compute q, waves 2-3 k.  Thread (16-byte channel segment c8, rows
// t0 .. t0 + RPT - 1 of its part) loads its RPT + 3 raw rows and the part's
// taps, and writes q -> Qc, k -> Kr (bf16 rows in LDS, zero past the sequence
// end).
// The loads are unconditional (rows clamped into x) so that they can all be
// in flight together; the few lanes whose window starts before the sequence
// replace those rows with the conv state after the loads have landed.
template <int D>
struct ConvRaw {
  static constexpr int RPT = kC * (D / 8) / 128;  // rows per thread (128 threads per part)
  uint4 x[RPT + 3];                               // raw rows t0 - 3 .. t0 + RPT - 1
};

// A per-head parameter stored as bf16 or fp32 (is_f32), read with two 16-bit
// loads whose addresses do not depend on a branch.
__device__ __forceinline__ float param_bits(const void* p, int h, int is_f32) {
  const uint16_t* q = static_cast<const uint16_t*>(p);
  const uint32_t hi = q[is_f32 ? 2 * h + 1 : h];
  const uint32_t lo = q[is_f32 ? 2 * h : h];
  return __uint_as_float((hi << 16) | (is_f32 ? lo : 0u));
}

__device__ __forceinline__ int conv_part_channel(const ConvIn& cv, int part, int kh, int h, int D) {
  return part == 0 ? kh * D : part == 1 ? cv.key_dim + kh * D : 2 * cv.key_dim + h * D;
}

template <int D>
__device__ __forceinline__ void conv_load(ConvRaw<D>& R, const ConvIn& cv, int part, int64_t tok0, int len, int kh,
                                          int h, int tid) {
  constexpr int SEG = D / 8;
  const int c8 = tid % SEG, t0 = ConvRaw<D>::RPT * (tid / SEG);
  const int ch = conv_part_channel(cv, part, kh, h, D) + 8 * c8;
  // chunk rows t >= lo keep row tok0 + t >= 0 (the clamp in 32 bits)
  const int lo = tok0 < 3 ? -static_cast<int>(tok0) : -3;
#pragma unroll
  for (int i = 0; i < ConvRaw<D>::RPT + 3; ++i) {
    // rows past the sequence end re-read its last row (outputs dropped); rows
    // before the first chunk's start are replaced by the state
    const int t = t0 - 3 + i;
    const int64_t row = tok0 + max(min(t, len - 1), lo);
    R.x[i] = *reinterpret_cast<const uint4*>(cv.x + row * cv.sx + ch);
  }
}

// Rows before the sequence's first token (row t0 - 3 + i < 0 of the first
// chunk): the conv state's tap t0 + i.
template <int D>
__device__ __forceinline__ void conv_state_halo(ConvRaw<D>& R, const ConvIn& cv, int part, bool first, int r,
                                                int kh, int h, int tid) {
  constexpr int SEG = D / 8;
  const int c8 = tid % SEG, t0 = ConvRaw<D>::RPT * (tid / SEG);
  if (first && t0 < 3) {
    if (cv.fresh && cv.fresh[r]) {  // a fresh sequence: zero state
#pragma unroll
      for (int i = 0; i < 3; ++i)
        if (t0 + i < 3) R.x[i] = make_uint4(0u, 0u, 0u, 0u);
      return;
    }
    const int64_t slot = cv.ids ? cv.ids[r] : r;
    const int ch = conv_part_channel(cv, part, kh, h, D) + 8 * c8;
    const uint16_t* sp = cv.cstate + slot * cv.ss_seq + static_cast<int64_t>(ch) * cv.ss_ch + t0;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (t0 + i >= 3) break;
      uint32_t u[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        u[e] = static_cast<uint32_t>(sp[static_cast<int64_t>(2 * e) * cv.ss_ch + i]) |
               (static_cast<uint32_t>(sp[static_cast<int64_t>(2 * e + 1) * cv.ss_ch + i]) << 16);
      R.x[i] = make_uint4(u[0], u[1], u[2], u[3]);
    }
  }
}

__device__ __forceinline__ float bf_elem(const uint4& u, int e) {
  const uint32_t w = e < 2 ? u.x : e < 4 ? u.y : e < 6 ? u.z : u.w;
  return (e & 1) ? hi_half(w) : lo_half(w);
}

template <int D>
__device__ __forceinline__ void conv_compute(const ConvRaw<D>& R, const ConvIn& cv, int part, uint16_t (*Qc)[D + 8],
                                             uint16_t (*Kr)[D + 8], int64_t tok0, int len, int kh, int h, int Hv,
                                             int tid) {
  constexpr int SEG = D / 8;
  constexpr int RPT = ConvRaw<D>::RPT;
  const int c8 = tid % SEG, t0 = RPT * (tid / SEG);
  // the part's taps (8 channels x 4), read here rather than with the rows:
  // every workgroup reads the same few KiB, so they come from cache
  uint4 wt[4];
  {
    const uint4* wp =
        reinterpret_cast<const uint4*>(cv.w + static_cast<int64_t>(conv_part_channel(cv, part, kh, h, D) + 8 * c8) * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) wt[j] = wp[j];
  }
  // two channels at a time keep the unpacked window small
  uint32_t yp[RPT][4];
#pragma unroll
  for (int e2 = 0; e2 < 4; ++e2) {
    float y[2][RPT];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int e = 2 * e2 + c;
      float wk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) wk[j] = bf_elem(wt[(4 * e + j) / 8], (4 * e + j) % 8);
      float xe[RPT + 3];
#pragma unroll
      for (int i = 0; i < RPT + 3; ++i) xe[i] = bf_elem(R.x[i], e);
#pragma unroll
      for (int rr = 0; rr < RPT; ++rr) y[c][rr] = gdn::conv4_silu(xe[rr], xe[rr + 1], xe[rr + 2], xe[rr + 3], wk);
    }
#pragma unroll
    for (int rr = 0; rr < RPT; ++rr) yp[rr][e2] = gdn::f2bf2(y[0][rr], y[1][rr]);
  }
#pragma unroll
  for (int rr = 0; rr < RPT; ++rr) {
    const int t = t0 + rr;
    u32x4_t out = {yp[rr][0], yp[rr][1], yp[rr][2], yp[rr][3]};
    if (len < kC && t >= len) out = u32x4_t{0u, 0u, 0u, 0u};  // only a sequence's last chunk
    *reinterpret_cast<u32x4_t*>(part == 0 ? &Qc[t][8 * c8] : &Kr[t][8 * c8]) = out;
  }
}

// Waves 0-1 compute the q part, waves 2-3 the k part (wave-uniform).
template <int D>
__device__ __forceinline__ void conv_chunk_rows(const ConvIn& cv, uint16_t (*Qc)[D + 8], uint16_t (*Kr)[D + 8],
                                                int64_t tok0, int len, bool first, int r, int kh, int h, int Hv,
                                                int tid) {
  const int part = __builtin_amdgcn_readfirstlane(tid >> 7);
  const int ptid = tid & 127;
  ConvRaw<D> R;
  conv_load<D>(R, cv, part, tok0, len, kh, h, ptid);
  gdn::keep_loads_here();
  conv_state_halo<D>(R, cv, part, first, r, kh, h, ptid);
  conv_compute<D>(R, cv, part, Qc, Kr, tok0, len, kh, h, Hv, ptid);
}

// grid = 8 * ceil(nc_bound * Hv / kR / 8); block = 256.  One workgroup per
// (chunk, kR value heads of one key head); writes the chunk's record of each.
// kR = 1, or 2 when Hv = 2 Hk (every value head of a key head).
// kConv: q, k are the conv1d + SiLU of cv.x and g, beta the gates of cv.a,
// cv.b, all computed here (the q, k, g, beta arguments unused).
template <int D, bool kConv, int kR>
__global__ __launch_bounds__(256, 4) void chunk_prep_kernel(
    const uint16_t* __restrict__ q, int64_t sq, const uint16_t* __restrict__ k, int64_t sk,
    const float* __restrict__ g, const uint16_t* __restrict__ beta, const int64_t* __restrict__ cu,
    int n_seqs, int64_t nc_bound, int Hk, int Hv, float scale, int l2norm, uint8_t* __restrict__ ws,
    ConvIn cv) {
  constexpr int NW = 4;
  constexpr int NT = 64 * NW;
  constexpr int KTD = D / 32;
  constexpr int SEG = D / 8;            // 16-byte segments per row
  constexpr int NSEG1 = kC * SEG / NT;  // row segments per thread
  static_assert(kC * SEG % NT == 0 && NT % SEG == 0, "segment tiling");
  __shared__ PrepSmem<D> sm;

  // One workgroup per (chunk, kR value heads of one key head): the q and k
  // rows, their conv and their sums of squares are the key head's; with kR =
  // 2 the two value heads then run one after the other, each writing its own
  // record, so the shared part runs once per key head.
  const int64_t wi = gdn::xcd_remap(blockIdx.x, nc_bound * (Hv / kR));
  if (wi < 0) return;
  const int64_t cidx = wi / (Hv / kR);
  int h = static_cast<int>(wi % (Hv / kR)) * kR;  // the value head in hand
  const int kh = h / (Hv / Hk);
  int r;
  int64_t jc;
  if (!locate_chunk(cu, n_seqs, cidx, &r, &jc)) return;
  const int64_t tok0 = cu[r] + jc * kC;
  const int len = static_cast<int>(min<int64_t>(kC, cu[r + 1] - tok0));
  const uint16_t* qh = q + static_cast<int64_t>(kh) * D;
  const uint16_t* kh_ = k + static_cast<int64_t>(kh) * D;
  uint8_t* rec = ws + (cidx * Hv + h) * rec_bytes(D);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int lr = lane & 15;
  const int lg = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- phase 1: K rows, row norms of K and Q, gates ----
  // q is held straight in the layout in which it serves as the A blocks' B
  // operand: wave w holds query rows 16 w + lr, keys 32 kk + 8 lg.  The same
  // registers become Q' once cQ is known.  The fused variant first runs the
  // conv into LDS (q rows in the L / T tiles' space, free until phase 2a).
  uint16_t (*Qc)[D + 8] = reinterpret_cast<uint16_t (*)[D + 8]>(&sm.Lp[0][0][0]);
  static_assert(sizeof(sm.Lp) + sizeof(sm.Td) >= sizeof(uint16_t) * kC * (D + 8), "conv q rows fit L and T");
  s16x8_t qv[KTD];
  auto q_rows = [&]() {
    const int t = 16 * wave + lr;
    if constexpr (kConv) {
#pragma unroll
      for (int kk = 0; kk < KTD; ++kk) qv[kk] = *reinterpret_cast<const s16x8_t*>(&Qc[t][32 * kk + 8 * lg]);
    } else {
#pragma unroll
      for (int kk = 0; kk < KTD; ++kk) {
        qv[kk] = *reinterpret_cast<const s16x8_t*>(qh + (tok0 + min(t, len - 1)) * sq + 8 * lg + 32 * kk);
        if (t >= len) qv[kk] = s16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  };
  if constexpr (!kConv) q_rows();
  // gate inputs of token tok0 + lane and value head hh (used by wave 0),
  // loaded ahead of their use by every wave with in-range addresses, so no
  // load waits on a branch
  auto gate_in = [&](int hh, float& gi_, float& bi_, float& al_, float& dt_) {
    const int64_t gi = (tok0 + min(lane, len - 1)) * Hv + hh;
    if constexpr (kConv) {
      gi_ = gdn::bf2f(cv.a[gi]);
      bi_ = gdn::bf2f(cv.b[gi]);
      al_ = param_bits(cv.A_log, hh, cv.param_f32);
      dt_ = param_bits(cv.dt_bias, hh, cv.param_f32);
    } else {
      gi_ = g[gi];
      bi_ = gdn::bf2f(beta[gi]);
    }
  };
  // wave 0: the gates' cumulative log-decay G and beta of the chunk's tokens
  auto gates = [&](float gi_, float bi_, float al_, float dt_) {
    if (wave == 0) {
      float gv = 0.f, bv = 0.f;
      if (lane < len) {
        if constexpr (kConv) {
          gv = gdn::gate_g(gi_, al_, dt_);
          bv = gdn::bf2f(gdn::gate_beta(bi_));
        } else {
          gv = gi_;
          bv = bi_;
        }
      }
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float o_ = __shfl_up(gv, d, 64);
        if (lane >= d) gv += o_;
      }
      sm.G[lane] = gv;
      sm.bt[lane] = bv;
    }
  };
  float gin, bin, al = 0.f, dtb = 0.f;
  gate_in(h, gin, bin, al, dtb);
  gdn::keep_loads_here();
  if constexpr (kConv) {
    conv_chunk_rows<D>(cv, Qc, sm.u.Kr, tok0, len, jc == 0, r, kh, h, Hv, tid);
  } else {
#pragma unroll
    for (int j = 0; j < NSEG1; ++j) {
      const int e = tid + NT * j;
      const int t = e / SEG, c8 = e % SEG;
      const int64_t row = tok0 + min(t, len - 1);
      s16x8_t kv8 = *reinterpret_cast<const s16x8_t*>(kh_ + row * sk + c8 * 8);
      if (t >= len) kv8 = s16x8_t{0, 0, 0, 0, 0, 0, 0, 0};
      *reinterpret_cast<s16x8_t*>(&sm.u.Kr[t][c8 * 8]) = kv8;
    }
  }
  gates(gin, bin, al, dtb);
  if constexpr (kConv) {
    __syncthreads();  // the conv's q rows are in LDS
    q_rows();
  }
  __syncthreads();

  // ---- the rows' sums of squares: the diagonals of the Gram tiles K K^T and
  //      Q Q^T of wave w's 16 rows (the bf16 products are exact; the matrix
  //      core sums them in fp32).  A row's A and B operand fragments are the
  //      same registers, so Q Q^T needs no LDS read.  C lane (column lr, rows
  //      4 lg + i) holds the diagonal element (lr, lr) at lg = lr / 4,
  //      i = lr % 4. ----
  {
    const int t = 16 * wave + lr;
    f32x4_t gk = {0.f, 0.f, 0.f, 0.f}, gq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KTD; ++kk) {
      const s16x8_t k8 = *reinterpret_cast<const s16x8_t*>(&sm.u.Kr[t][32 * kk + 8 * lg]);
      gk = gdn::mfma16x16x32(k8, k8, gk);
      gq = gdn::mfma16x16x32(qv[kk], qv[kk], gq);
    }
    if (lg == (lr >> 2)) {
      const int i = lr & 3;
      sm.ssk[t] = i == 0 ? gk[0] : i == 1 ? gk[1] : i == 2 ? gk[2] : gk[3];
      sm.ssq[t] = i == 0 ? gq[0] : i == 1 ? gq[1] : i == 2 ? gq[2] : gq[3];
    }
  }
  __syncthreads();

  // The K rows, kept in registers for the value heads after the first (the
  // solve reuses their LDS bytes), and the loop over the key head's value
  // heads; each writes its record (h, rec), the next one's gate inputs loaded
  // one head ahead.
  s16x8_t kkeep[NSEG1];
  if constexpr (kR > 1) {
#pragma unroll
    for (int j = 0; j < NSEG1; ++j) {
      const int e = tid + NT * j;
      kkeep[j] = *reinterpret_cast<const s16x8_t*>(&sm.u.Kr[e / SEG][(e % SEG) * 8]);
    }
  }
  float ngin = 0.f, nbin = 0.f, nal = 0.f, ndtb = 0.f;
#pragma unroll
  for (int rr = 0; rr < kR; ++rr) {
  if (rr > 0) {
    ++h;
    rec += rec_bytes(D);
#pragma unroll
    for (int j = 0; j < NSEG1; ++j) {
      const int e = tid + NT * j;
      *reinterpret_cast<s16x8_t*>(&sm.u.Kr[e / SEG][(e % SEG) * 8]) = kkeep[j];
    }
    gates(ngin, nbin, nal, ndtb);
    __syncthreads();
  }
  if (rr + 1 < kR) gate_in(h + 1, ngin, nbin, nal, ndtb);

  // ---- K^T (as soon as the K rows are in LDS, so its stores retire during
  //      the solve), key tile kt = wave, by a bf16 identity product C = K I
  //      with the identity's columns qswap-ordered: lane (position n, g) of C holds
  //      key qswap(32 kt + n) at tokens 8i + 4g + r, i.e. at token positions
  //      8g + 0..7 (elements 0..7) and 16 + 8g + 0..7 (elements 8..15); the
  //      product is exact, the fp16 packing rounds K once. ----
  if (wave < D / 32) {
    const int kt = wave;
    const int li = lane & 31, g = lane >> 5;
    const s16x8_t iq0 = ident_frag(0, qswap(li), g), iq1 = ident_frag(1, qswap(li), g);
    uint8_t* kp = rec + rec_kt(D);
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const s16x8_t* kr = reinterpret_cast<const s16x8_t*>(&sm.u.Kr[32 * tt + li][32 * kt + 8 * g]);
      f32x16_t kc = mfma32_bf16(kr[0], iq0, zero16());
      kc = mfma32_bf16(kr[2], iq1, kc);
      *reinterpret_cast<h16x8_t*>(kp + frag_byte(kt * 4 + 2 * tt, lane)) = pack_h8<0>(kc);
      *reinterpret_cast<h16x8_t*>(kp + frag_byte(kt * 4 + 2 * tt + 1, lane)) = pack_h8<8>(kc);
    }
  }

  if (tid < kC) {
    const int t = tid;
    // rk = 0 past the sequence end: cK and T' then clear those key tokens
    const float rk = t < len ? (l2norm ? rsqrtf(sm.ssk[t] + 1e-6f) : 1.0f) : 0.f;
    const float rq = l2norm ? rsqrtf(sm.ssq[t] + 1e-6f) : 1.0f;
    const float Gt = sm.G[t];
    const float Gl = sm.G[kC - 1];
    sm.rk[t] = rk;
    sm.rq[t] = rq;
    const float cqv = rq * scale * expf(Gt);
    sm.cq[t] = cqv;
    float* vec = reinterpret_cast<float*>(rec + Rec::VEC);
    vec[t] = cqv;
    vec[kC + t] = rk * expf(Gl - Gt);
    vec[Rec::CT + t] = -(rk * expf(Gt));
    if (t == 0) vec[2 * kC] = expf(Gl);
  }
  __syncthreads();

  // ---- Q' = diag(cQ) q as fp16, in B-fragment order: this lane's keys
  //      32 kk + 8 lg of token t are fragment (t / 32, 2 kk + lg / 2), lane
  //      t % 32 + 32 (lg % 2) ----
  {
    uint8_t* qrec = rec + Rec::QP;
    const int t = 16 * wave + lr;
    const float cqv = sm.cq[t];
#pragma unroll
    for (int kk = 0; kk < KTD; ++kk) {
      const u32x4_t x = __builtin_bit_cast(u32x4_t, qv[kk]);
      u32x4_t y;
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = f2h2(lo_half(x[i]) * cqv, hi_half(x[i]) * cqv);
      const int frag = (t >> 5) * (D / 16) + 2 * kk + (lg >> 1);
      *reinterpret_cast<u32x4_t*>(qrec + frag_byte(frag, (t & 31) + 32 * (lg & 1))) = y;
    }
  }

  // ---- phase 2a: K K^T -> L (fp32 lower tiles) ----
  for (int j = wave; j < 10; j += NW) {
    int mt, nt;
    tri_tile(j, mt, nt);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KTD; ++kk) {
      const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.u.Kr[16 * mt + lr][32 * kk + 8 * lg]);
      const s16x8_t b8 = *reinterpret_cast<const s16x8_t*>(&sm.u.Kr[16 * nt + lr][32 * kk + 8 * lg]);
      acc = gdn::mfma16x16x32(a8, b8, acc);
    }
    const int s = 16 * nt + lr;
    const float rks = sm.rk[s];
    const float Gs = sm.G[s];
    // rows t = 16 mt + 4 lg + i: four consecutive tokens, one 16-byte read per vector
    const int t0 = 16 * mt + 4 * lg;
    const float4 btv = *reinterpret_cast<const float4*>(&sm.bt[t0]);
    const float4 rkv = *reinterpret_cast<const float4*>(&sm.rk[t0]);
    const float4 gv = *reinterpret_cast<const float4*>(&sm.G[t0]);
    const float bt4[4] = {btv.x, btv.y, btv.z, btv.w}, rk4[4] = {rkv.x, rkv.y, rkv.z, rkv.w};
    const float g4[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float l = acc[i] * bt4[i] * rk4[i] * rks * __expf(g4[i] - Gs);
      // below the diagonal tile every s < t; on it the strict lower triangle
      sm.Lp[j][4 * lg + i][lr] = (mt != nt || s < t0 + i) ? l : 0.f;
    }
  }
  __syncthreads();

  // ---- phase 2b: wave 0 inverts the diagonal blocks; every wave w forms the
  //      rows 16 w .. 16 w + 15 of A = lower_incl(scale q^.k^ e^{G_t - G_s})
  //      from the q rows it holds, and writes them to the record ----
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
    for (int rr = 0; rr < 16; ++rr) sm.Td[bb][rr][c] = x[rr];
  }
  {
    // key-token tiles ns of the 32-wide column blocks the rows touch; tiles
    // above the diagonal are written as zeros
    uint8_t* arec = rec + Rec::AQ;
    const int mt = wave;
    const int t = 16 * mt + lr;  // the lane's query token (C column)
    const float qscale = sm.rq[t] * scale;
    const float Gt = sm.G[t];
#pragma unroll 1
    for (int ns = 0; ns <= (mt | 1); ++ns) {  // wave-uniform trip count
      float a[4] = {0.f, 0.f, 0.f, 0.f};       // tiles above the diagonal stay zero
      if (ns <= mt) {
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KTD; ++kk) {
          const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.u.Kr[16 * ns + lr][32 * kk + 8 * lg]);
          acc = gdn::mfma16x16x32(a8, qv[kk], acc);
        }
        // keys s = 16 ns + 4 lg + i: four consecutive tokens
        const int s0 = 16 * ns + 4 * lg;
        const float4 rkv = *reinterpret_cast<const float4*>(&sm.rk[s0]);
        const float4 gv = *reinterpret_cast<const float4*>(&sm.G[s0]);
        const float rk4[4] = {rkv.x, rkv.y, rkv.z, rkv.w}, g4[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float av = acc[i] * qscale * rk4[i] * __expf(Gt - g4[i]);
          a[i] = ((ns < mt || s0 + i <= t) && t < len) ? av : 0.f;
        }
      }
      // tokens 16 ns + 4 lg .. + 3 sit at the positions of quad qswap
      const int pos = qswap(16 * ns + 4 * lg);
      uint2 pk, lo;
      pk.x = f2h2(a[0], a[1]);
      pk.y = f2h2(a[2], a[3]);
      lo.x = f2h2_lo(a[0], a[1], pk.x);
      lo.y = f2h2_lo(a[2], a[3], pk.y);
      *reinterpret_cast<uint2*>(arec + tri_frag_byte(t, pos)) = pk;
      *reinterpret_cast<uint2*>(arec + (Rec::AL - Rec::AQ) + tri_frag_byte(t, pos)) = lo;
    }
  }
  __syncthreads();
  // first sub-diagonal: T(j+1, j) = -T(j+1,j+1) L(j+1,j) T(j,j)
  if (wave < 3) {
    const int j = wave, i = j + 1;
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(i, j)][0][0], kTileLd, t_tile(sm, j, j), kTileLd, lane);
    st16_f32(&sm.u.s.scr[wave][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, t_tile(sm, i, i), kTileLd, &sm.u.s.scr[wave][0][0], kTileLd, lane);
    st16_f32(t_tile(sm, i, j), t2, -1.f, lane);
  } else {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(3, 0)][0][0], kTileLd, t_tile(sm, 0, 0), kTileLd, lane);  // L30 T00
    st16_f32(&sm.u.s.scr[3][0][0], p, 1.f, lane);
  }
  __syncthreads();
  // second sub-diagonal: T20, T31; partial sum for T30
  if (wave == 0) {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(2, 0)][0][0], kTileLd, t_tile(sm, 0, 0), kTileLd, lane);  // L20 T00
    p = mm16_f32(p, &sm.Lp[tix(2, 1)][0][0], kTileLd, t_tile(sm, 1, 0), kTileLd, lane);  // L21 T10
    st16_f32(&sm.u.s.scr[0][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, t_tile(sm, 2, 2), kTileLd, &sm.u.s.scr[0][0][0], kTileLd, lane);
    st16_f32(t_tile(sm, 2, 0), t2, -1.f, lane);
  } else if (wave == 1) {
    f32x4_t p = {0.f, 0.f, 0.f, 0.f};
    p = mm16_f32(p, &sm.Lp[tix(3, 1)][0][0], kTileLd, t_tile(sm, 1, 1), kTileLd, lane);  // L31 T11
    p = mm16_f32(p, &sm.Lp[tix(3, 2)][0][0], kTileLd, t_tile(sm, 2, 1), kTileLd, lane);  // L32 T21
    st16_f32(&sm.u.s.scr[1][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, t_tile(sm, 3, 3), kTileLd, &sm.u.s.scr[1][0][0], kTileLd, lane);
    st16_f32(t_tile(sm, 3, 1), t2, -1.f, lane);
  } else if (wave == 3) {
    f32x4_t p = ld16_f32(&sm.u.s.scr[3][0][0], lane);
    p = mm16_f32(p, &sm.Lp[tix(3, 1)][0][0], kTileLd, t_tile(sm, 1, 0), kTileLd, lane);  // + L31 T10
    st16_f32(&sm.u.s.scr[3][0][0], p, 1.f, lane);
  }
  __syncthreads();
  // third sub-diagonal: T30
  if (wave == 3) {
    f32x4_t p = ld16_f32(&sm.u.s.scr[3][0][0], lane);
    p = mm16_f32(p, &sm.Lp[tix(3, 2)][0][0], kTileLd, t_tile(sm, 2, 0), kTileLd, lane);  // + L32 T20
    st16_f32(&sm.u.s.scr[3][0][0], p, 1.f, lane);
    wave_sync();
    f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
    t2 = mm16_f32(t2, t_tile(sm, 3, 3), kTileLd, &sm.u.s.scr[3][0][0], kTileLd, lane);
    st16_f32(t_tile(sm, 3, 0), t2, -1.f, lane);
  }
  __syncthreads();

  // ---- T'' = T diag(beta): fp16 granules of 8 column positions (two token
  //      quads each) ----
  for (int e = tid; e < kC * 8; e += NT) {
    const int t = (e >> 3) & 63, gp = e & 7;
    if ((gp >> 2) > (t >> 5)) continue;  // above the diagonal blocks: not stored
    const float4 a = t_quad(sm, sm.bt, t, quad_of_pos(2 * gp));
    const float4 b = t_quad(sm, sm.bt, t, quad_of_pos(2 * gp + 1));
    uint4 pk;
    pk.x = f2h2(a.x, a.y);
    pk.y = f2h2(a.z, a.w);
    pk.z = f2h2(b.x, b.y);
    pk.w = f2h2(b.z, b.w);
    *reinterpret_cast<uint4*>(rec + Rec::TB + tri_frag_byte(t, 8 * gp)) = pk;
  }
  // the T tiles and gates are read before the next value head's K rows and
  // gates overwrite them
  if (rr + 1 < kR) __syncthreads();
  }
}

// ============================================================ state kernel ==
template <int D>
struct __align__(16) StateStage {
  h16x8_t Kt[D / 32 * 4][64];  // K^T fragments [key tile * 4 + token step][lane]; rows in
                                // position order (row p holds key qswap(p))
  h16x8_t W[2 * (D / 16)][64];  // -W fragments [token tile * D/16 + key step][lane]
  s16x8_t Vc[2][2][2][64];      // V (bf16) [column tile][token tile][16-column half][lane]: A operands of V^T = V I
  h16x8_t Tb[6][64];            // T'' fragments (A operands of U = T'' V)
  float vec[256];               // record VEC: cQ[64], cK[64], e^gamma
};

// What the chain waves hand the output waves, in register order: the fp16
// operand fragments of S before the chunk's update (one buffer: the output
// waves read it in the same barrier interval, after the chain wave's flag
// says it is there), and of Vn as a rounded part and its rounding residual
// (Vn = Vh + Vl to ~22 significant bits; two buffers: the output waves use
// them one interval later).
template <int D>
struct __align__(16) StateXchgS {
  h16x8_t Sh[2][D / 16][64];
};
struct __align__(16) StateXchgV {
  h16x8_t Vh[2][4][64];
  h16x8_t Vl[2][4][64];
};

template <int D>
struct __align__(16) StateSmem {
  StateStage<D> st[2];
  StateXchgS<D> xs;
  StateXchgV xv[2];
  uint16_t ot[2][32 * kCB];  // each output wave's bf16 tile on its way out, swz<64>
  uint16_t vtile[2][67 * 16];  // fused: each U wave's conv window rows (one k-step's 16 channels)
  float vw[2][32 * 4];         // fused: each U wave's 32 channels' conv taps (fp32)
  int sflag[2][64];            // chain wave w: chunks whose S it has put in xs (sflag[w][*] = j + 1)
};

constexpr int kStateWaves = 8;

// Wave roles of the state kernel (wave w; waves land on the SIMDs in the
// order 0, 2, 1, 3, 0, 2, 1, 3 or a rotation of it, so waves w and w + 4
// share a SIMD: each chain wave shares with a K wave, each output wave with a
// U wave, whose VALU-heavy conv (fused variant) stays off the chain's SIMDs):
//   w 0, 1  chain: the recurrence for state columns 32 w .. 32 w + 31 of the
//           workgroup's 64 (Vn = U - W S, S <- e^gamma S + K^T diag(cK) Vn)
//   w 2, 3  output: O^T = S^T Q'^T + Vn^T A^T of token tile w - 2 (both
//           chains' columns): S^T Q'^T in the chain's interval (once the
//           chain waves' flags show S), Vn^T A^T in the next one, as three
//           fp16 products (Vh A + Vl A + Vh A_lo) that carry Vn and A to ~22
//           significant bits
//   w 4, 5  K: the record's K^T and -W = -T' K for key tiles w - 4 (+ 2), the
//           record's vec block and T'' (three fragments each), into the stage
//   w 6, 7  U: V of value-column tile w - 6 into the stage (fused variant: V
//           is the conv1d + SiLU of the raw v channels, computed here); the
//           chain wave of those columns forms V^T and U = T'' V at the start
//           of its interval
// Per chunk the chain, U, output and K roles issue 42, 0, 40 and 12
// matrix-core products of 32x32x16.  A 32-column workgroup (one tile) runs
// chain wave 0 only (wave 1 takes part in the barriers), output waves on one
// accumulation chain each (20 products), and U waves 6 and 7 on one 16-column
// half of the tile each.

// Per-lane prefetch registers of one chunk, one struct per role.
template <int D>
struct KPrefetch {
  static constexpr int NKT = D / 64;  // key tiles per K wave: pk, pk + 2
  s16x8_t k[NKT][4];                  // K^T fragments: key tile pk + 2u, token step
  s16x8_t tw[6];                      // the six T'' fragments (scaled into -T' by k_stage)
  s16x8_t vec;                        // the lane's 16 bytes of the record vec block
};

// Conv inputs of the fused variant: the U waves compute the conv1d + SiLU of
// their v channels from the raw rows, and the output waves roll the conv state.
struct StateConv {
  const uint16_t* x;  // [N, C] raw rows, row stride sx (NULL: not fused)
  int64_t sx;
  uint16_t* cstate;   // conv state pool: row slot, channel c, tap j at cstate + slot*ss_seq + c*ss_ch + j
  int64_t ss_seq, ss_ch;
  const uint16_t* w;  // [C, 4] conv taps
  int key_dim;        // Hk * D; the v channels start at 2 key_dim
  int ratio;          // Hv / Hk
};

struct UPrefetch {
  s16x8_t v[2][2];  // V rows (fused: raw rows): token tile tt, the wave's value k-step i (NH of them)
};

template <int D>
struct QPrefetch {
  s16x8_t q[D / 16];  // Q' fragments of the wave's token tile, per key step
};
struct APrefetch {
  s16x8_t a[4];   // A fragments 2 nt .. 2 nt + 3: k-steps 0..1 of tile 0, 0..3 of tile 1
  s16x8_t al[4];  // the same fragments of A's residual
};

// Raw buffer access: a wave-uniform base in the descriptor, the per-lane
// byte offset in a VGPR that stays fixed across chunks, and the per-load part
// in the scalar offset, so the prefetches need no per-load address registers.
// The range is left open (offsets are computed in bounds); the third word is
// the gfx9 raw-dword format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ s16x8_t buf_ld(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(s16x8_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// The prefetches issue the loads of one chunk for this lane.  Nothing here
// consumes a loaded value, so the loads stay in flight until staging.
// K^T fragments and the vec block, then the -T' fragments.
template <int D>
__device__ __forceinline__ void k_prefetch_kt(KPrefetch<D>& p, const uint8_t* rec, int pk, int lane) {
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(rec);
  const int kt0 = static_cast<int>(rec_kt(D));
#pragma unroll
  for (int u = 0; u < KPrefetch<D>::NKT; ++u)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) p.k[u][ks] = buf_ld(r, 16 * lane, kt0 + 1024 * ((pk + 2 * u) * 4 + ks));
  p.vec = buf_ld(r, 16 * lane, Rec::VEC);
}

template <int D>
__device__ __forceinline__ void k_prefetch_tw(KPrefetch<D>& p, const uint8_t* rec, int pk, int lane) {
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(rec);
#pragma unroll
  for (int j = 0; j < 6; ++j) p.tw[j] = buf_ld(r, 16 * lane, Rec::TB + 1024 * j);
}

// V rows past the sequence end re-read its last token: those tokens carry
// zero weights in T'', and their outputs are not stored.
// (NH 16-column halves of tile c from half hb on: both halves in a
// 64-column workgroup, one per U wave in a 32-column one)
template <int NH>
__device__ __forceinline__ void u_prefetch(UPrefetch& p, const uint16_t* vh, int sv, int64_t tok0, int len, int c,
                                           int hb, int lane) {
  const int li = lane & 31, g = lane >> 5;
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vh + tok0 * sv);
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int off = 2 * (min(32 * tt + li, len - 1) * sv + 32 * c + 8 * g);
#pragma unroll
    for (int i = 0; i < NH; ++i) p.v[tt][i] = buf_ld(rv, off, 32 * (hb + i));
  }
}

template <int D>
__device__ __forceinline__ void q_prefetch(QPrefetch<D>& p, const uint8_t* rec, int nt, int lane) {
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(rec);
#pragma unroll
  for (int s = 0; s < D / 16; ++s) p.q[s] = buf_ld(r, 16 * lane, Rec::QP + 1024 * (nt * (D / 16) + s));
}

// the fragments of token tile NT: key steps 0..1 for tile 0, 0..3 for tile 1
// (the output role is compiled per tile, so each path's loads are exact)
template <int NT>
__device__ __forceinline__ void a_prefetch(APrefetch& p, const uint8_t* rec, int lane) {
  constexpr int NA = NT ? 4 : 2;
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(rec);
#pragma unroll
  for (int ks = 0; ks < NA; ++ks) p.a[ks] = buf_ld(r, 16 * lane, Rec::AQ + 1024 * (2 * NT + ks));
#pragma unroll
  for (int ks = 0; ks < NA; ++ks) p.al[ks] = buf_ld(r, 16 * lane, Rec::AL + 1024 * (2 * NT + ks));
}

// K waves: K^T and -W of key tiles pk (+ 2) into the stage, as fragments.
// -W^T = K^T (-T')^T with the record's fp16 K^T fragments as A operands: lane
// (token t, g) of its C tiles holds keys 32 kt + 8g + 0..7 and
// 32 kt + 16 + 8g + 0..7, the -W fragments of key steps 2 kt, 2 kt + 1.  The
// K^T fragments themselves are the state update's A operands.
template <int D>
__device__ __forceinline__ void k_stage(KPrefetch<D>& p, StateStage<D>& S, int pk, int lane,
                                        const uint8_t* next_rec) {
  constexpr int KS = D / 16;
  constexpr int NKT = KPrefetch<D>::NKT;
  *reinterpret_cast<s16x8_t*>(reinterpret_cast<uint8_t*>(S.vec) + 16 * lane) = p.vec;
  // this wave's three of the six T'' fragments into the stage, as they are
  if (pk == 0) {
#pragma unroll
    for (int j = 0; j < 3; ++j) S.Tb[j][lane] = as_h8(p.tw[j]);
  } else {
#pragma unroll
    for (int j = 0; j < 3; ++j) S.Tb[3 + j][lane] = as_h8(p.tw[j + 3]);
  }
  // -T' = T'' diag(cT): lane group g's element e of k-step ks is token
  // 16 ks + 4 g + e (e < 4) or 16 ks + 8 + 4 g + e - 4, whose cT this wave
  // has just written to the stage's vec block (its own LDS writes, in order)
  {
    const int g = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const float4 fa = *reinterpret_cast<const float4*>(&S.vec[Rec::CT + 16 * ks + 4 * g]);
      const float4 fb = *reinterpret_cast<const float4*>(&S.vec[Rec::CT + 16 * ks + 8 + 4 * g]);
      const float f[8] = {fa.x, fa.y, fa.z, fa.w, fb.x, fb.y, fb.z, fb.w};
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        if (jj == 0 && ks >= 2) continue;     // (row tile 0 has k-steps 0..1 only)
        const int j = jj == 0 ? ks : ks + 2;
        const h16x8_t t8 = as_h8(p.tw[j]);
        h16x8_t w8;
#pragma unroll
        for (int e = 0; e < 8; ++e) w8[e] = static_cast<_Float16>(static_cast<float>(t8[e]) * f[e]);
        p.tw[j] = __builtin_bit_cast(s16x8_t, w8);
      }
    }
  }
  f32x16_t cw[NKT][2];
#pragma unroll
  for (int u = 0; u < NKT; ++u) {
    const int kt = pk + 2 * u;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) S.Kt[kt * 4 + ks][lane] = as_h8(p.k[u][ks]);
    cw[u][0] = mfma32(as_h8(p.k[u][0]), as_h8(p.tw[0]), zero16());
    cw[u][1] = mfma32(as_h8(p.k[u][0]), as_h8(p.tw[2]), zero16());
    cw[u][0] = mfma32(as_h8(p.k[u][1]), as_h8(p.tw[1]), cw[u][0]);
    cw[u][1] = mfma32(as_h8(p.k[u][1]), as_h8(p.tw[3]), cw[u][1]);
    cw[u][1] = mfma32(as_h8(p.k[u][2]), as_h8(p.tw[4]), cw[u][1]);
    cw[u][1] = mfma32(as_h8(p.k[u][3]), as_h8(p.tw[5]), cw[u][1]);
  }
  // The next chunk's loads go out as soon as these registers are read: a
  // single set of registers then carries a whole iteration's worth of loads.
  k_prefetch_kt<D>(p, next_rec, pk, lane);
  k_prefetch_tw<D>(p, next_rec, pk, lane);
  gdn::keep_loads_here();
#pragma unroll
  for (int u = 0; u < NKT; ++u) {
    const int kt = pk + 2 * u;
    S.W[2 * kt][lane] = pack_h8<0>(cw[u][0]);
    S.W[2 * kt + 1][lane] = pack_h8<8>(cw[u][0]);
    S.W[KS + 2 * kt][lane] = pack_h8<0>(cw[u][1]);
    S.W[KS + 2 * kt + 1][lane] = pack_h8<8>(cw[u][1]);
  }
}

// Fused variant: the conv1d + SiLU of the lane's V elements (token 32 tt + li,
// channels 32 c + 16 h + 8 g + 0..7) from the raw rows.  The window rows come
// through the wave's LDS tile (tile row i = chunk row i - 3, the 16 channels
// of one k-step h): the lanes' own rows, and in rows 0..2 the carry -- the
// previous chunk's last 3 rows, or before a sequence its conv state's taps.
// The carry for the next chunk is taken from the tile.  wt holds the 32
// channels' taps (fp32, 4 per channel).  Every conv goes through
// gdn::conv4_silu in the standalone kernel's operation order, so the values
// are bit-identical.
template <int NH>
__device__ __forceinline__ void u_conv(const UPrefetch& p, s16x8_t (&carry)[2], uint16_t* tile, const float* wt,
                                       int lane, s16x8_t (&vc)[2][2], int hb) {
  const int li = lane & 31, g = lane >> 5;
#pragma unroll
  for (int hs = 0; hs < NH; ++hs) {
    const int h = hb + hs;  // the half's 16 channels within the tile (register slot hs)
    *reinterpret_cast<s16x8_t*>(&tile[(3 + li) * 16 + 8 * g]) = p.v[0][hs];
    *reinterpret_cast<s16x8_t*>(&tile[(35 + li) * 16 + 8 * g]) = p.v[1][hs];
    if (li < 3) *reinterpret_cast<s16x8_t*>(&tile[li * 16 + 8 * g]) = carry[hs];
    wave_sync();
    uint4 x[2][3];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < 3; ++i) x[tt][i] = *reinterpret_cast<const uint4*>(&tile[(32 * tt + li + i) * 16 + 8 * g]);
    carry[hs] = *reinterpret_cast<const s16x8_t*>(&tile[(64 + min(li, 2)) * 16 + 8 * g]);
    uint32_t y[2][4];
#pragma unroll
    for (int e2 = 0; e2 < 4; ++e2) {
      float yy[2][2];
#pragma unroll
      for (int cc = 0; cc < 2; ++cc) {
        const int e = 2 * e2 + cc;
        const float4 w4 = reinterpret_cast<const float4*>(wt)[16 * h + 8 * g + e];
        const float wk[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          yy[tt][cc] = gdn::conv4_silu(bf_elem(x[tt][0], e), bf_elem(x[tt][1], e), bf_elem(x[tt][2], e),
                                       bf_elem(__builtin_bit_cast(uint4, p.v[tt][hs]), e), wk);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) y[tt][e2] = gdn::f2bf2(yy[tt][0], yy[tt][1]);
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) vc[tt][hs] = __builtin_bit_cast(s16x8_t, u32x4_t{y[tt][0], y[tt][1], y[tt][2], y[tt][3]});
    wave_sync();  // the tile is read before the next half's rows go in
  }
}

// U waves: V of column tile c (fused variant: the conv1d + SiLU of the raw
// v channels) into the stage as the A operands of V^T = V I, with the wave's
// three of T''s six fragments; the chain wave that owns the columns forms
// V^T and U = T'' V itself.
template <int D, bool kX, int NH>
__device__ __forceinline__ void u_stage(const UPrefetch& p, StateStage<D>& S, int c, int hb, int lane,
                                        s16x8_t (&carry)[2], uint16_t* tile, const float* wt) {
  s16x8_t vc[2][2];
  if constexpr (kX) {
    u_conv<NH>(p, carry, tile, wt, lane, vc, hb);
  } else {
#pragma unroll
    for (int tt = 0; tt < 2; ++tt)
#pragma unroll
      for (int i = 0; i < NH; ++i) vc[tt][i] = p.v[tt][i];
  }
#pragma unroll
  for (int tt = 0; tt < 2; ++tt)
#pragma unroll
    for (int i = 0; i < NH; ++i) S.Vc[c][tt][hb + i][lane] = vc[tt][i];
}

// Output waves, first half of a chunk: acc = S^T Q'^T for token tile nt and
// the 32 columns of each of the workgroup's NC chains (independent
// accumulation chains), once the chain waves have put the chunk's S in the
// exchange (flag >= j + 1).
// Each Q' register is reloaded from `next` (the chunk two ahead) right after
// its last product: one load between two products, so the wave's loads do not
// queue up in one burst at the address unit ahead of its products.
template <int D, int NC>
__device__ __forceinline__ void o_inter(QPrefetch<D>& p, const uint8_t* next, const StateXchgS<D>& X,
                                        const int* sflag, int64_t j, int nt, int lane, f32x16_t (&acc)[NC]) {
  constexpr int KS = D / 16;
  const int want = static_cast<int>(j) + 1;
  if constexpr (NC == 2) {
    while (min(__hip_atomic_load(&sflag[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP),
               __hip_atomic_load(&sflag[64], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < want)
      __builtin_amdgcn_s_sleep(1);
  } else {
    while (__hip_atomic_load(&sflag[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < want)
      __builtin_amdgcn_s_sleep(1);
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  h16x8_t sh[NC][KS];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int s = 0; s < KS; ++s) sh[c][s] = X.Sh[c][s][lane];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < NC; ++c) acc[c] = zero16();
  const __amdgpu_buffer_rsrc_t r = buf_rsrc(next);
#pragma unroll
  for (int s = 0; s < KS; ++s) {
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = mfma32(sh[c][s], as_h8(p.q[s]), acc[c]);
    __builtin_amdgcn_sched_barrier(0);
    p.q[s] = buf_ld(r, 16 * lane, Rec::QP + 1024 * (nt * KS + s));
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Output waves, second half (the interval after): acc += Vn^T A^T as
// Vh A + Vl A + Vh A_lo (o_intra), then the bf16 tile goes out (o_store).
// The A registers are reloaded after all of the products (a_prefetch).  Token
// tile 0 has A entries at token steps 0 and 1 only, tile 1 at 0..3; the role
// is compiled per tile (NT), so neither loads nor multiplies what is zero.
template <int NC, int NT>
__device__ __forceinline__ void o_intra(const APrefetch& p, const StateXchgV& X, f32x16_t (&acc)[NC], int lane) {
  constexpr int NS = NT ? 4 : 2;
  h16x8_t vh[NC][NS], vl[NC][NS];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      vh[c][s] = X.Vh[c][s][lane];
      vl[c][s] = X.Vl[c][s][lane];
    }
  __builtin_amdgcn_sched_barrier(0);
  // the residual products, then the rounded one
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = mfma32(vl[c][s], as_h8(p.a[s]), acc[c]);
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = mfma32(vh[c][s], as_h8(p.al[s]), acc[c]);
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = mfma32(vh[c][s], as_h8(p.a[s]), acc[c]);
}

// The C tiles give each lane 4 columns of a row per store; rows go out whole
// instead (the tile's 32 NC columns as 16-byte pieces, 4 NC lanes per row),
// through the wave's own LDS tile.  The caller issues the next chunk's A loads
// before this: gfx9 counts loads and stores on one counter, in order, so loads
// issued after the stores would not count as arrived before the stores had
// completed.
template <int NC>
__device__ __forceinline__ void o_store(const f32x16_t (&acc)[NC], uint16_t* ot, uint16_t* ob, int len, int Hv, int D,
                                        int nt, int lane) {
  constexpr int W = 32 * NC;       // tile columns
  constexpr int LPR = W / 8;       // lanes per row
  constexpr int RPI = 64 / LPR;    // rows per store instruction
  const int tl = lane & 31, g = lane >> 5;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x2_t pk;
      pk[0] = gdn::f2bf2(acc[c][4 * i], acc[c][4 * i + 1]);
      pk[1] = gdn::f2bf2(acc[c][4 * i + 2], acc[c][4 * i + 3]);
      *reinterpret_cast<u32x2_t*>(&ot[swz<W>(tl, 32 * c + 8 * i + 4 * g)]) = pk;
    }
  wave_sync();
  // Raw buffer stores whose range ends at the chunk's last token: rows past
  // the sequence end fall outside it and are dropped, so every path issues
  // the same stores.
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(ob, static_cast<short>(0), len * Hv * D * 2, 0x00020000);
  const int gr = lane % LPR;
#pragma unroll
  for (int u = 0; u < 32 / RPI; ++u) {
    const int row = RPI * u + lane / LPR;
    const u32x4_t x = *reinterpret_cast<const u32x4_t*>(&ot[swz<W>(row, 8 * gr)]);
    __builtin_amdgcn_raw_buffer_store_b128(x, r, 2 * ((32 * nt + row) * Hv * D + 8 * gr), 0, 0);
  }
  wave_sync();  // the tile is read before the next chunk's writes
}

// Conv-state roll of the fused variant, done here because the prep kernel
// reads the old q and k taps from every chunk-0 workgroup of a sequence (the
// value heads that share a key head included), and this kernel runs after all
// of them.  Workgroup (sequence r, value head h, columns col0 .. col0 +
// width - 1) rolls those v channels, and the q and k channels of its columns
// when h is the first value head of its key head: state taps j = 0..2 <- the raw inputs at
// positions T - 3 + j (old taps T + j where that is negative), as the
// standalone conv kernel does.  The output waves roll after the first
// workgroup barrier: the U waves read the v channels' old taps for their first
// chunk before it.
// (a fresh sequence rolls from a zero state: its old taps are not read)

template <int D>
__device__ __forceinline__ void conv_roll(const StateConv& cr, int64_t slot, bool fresh, int64_t bos, int64_t T, int h,
                                          int col0, int width, int i0, int nthreads) {
  const bool qk = h % cr.ratio == 0;
  const int kh = h / cr.ratio;
  const int ntask = (qk ? 3 : 1) * width;
  for (int task = i0; task < ntask; task += nthreads) {
    const int part = qk ? task / width : 2;
    const int ch = (part == 0 ? kh * D : part == 1 ? cr.key_dim + kh * D : 2 * cr.key_dim + h * D) + col0 +
                   task % width;
    uint16_t* st = cr.cstate + slot * cr.ss_seq + static_cast<int64_t>(ch) * cr.ss_ch;
    uint16_t val[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int64_t p = T - 3 + j;
      val[j] = p >= 0 ? cr.x[(bos + p) * cr.sx + ch] : (fresh ? static_cast<uint16_t>(0) : st[p + 3]);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) st[j] = gdn::roll_value(val[j]);
  }
}

// Segments of long sequences.  The state after chunk j is linear in the
// state before it: S' = A_j S + B_j with A_j = e^gamma I - K^T diag(cK) W and
// B_j = K^T diag(cK) U.  Over chunks [c0, c1) that gives S_c1 = P S_c0 + R,
// where R is the recurrence run from S = 0 and P the recurrence run on the
// identity's columns with U = 0.  A long sequence is cut into segments: the
// first runs as usual (outputs, from h0) and ends in the second's initial
// state; each middle segment runs once without outputs, in parallel with the
// first: its chain waves run R and its output waves, idle otherwise, run P on
// the same staged records; a scan S_{s+1} = P_s S_s + R_s gives every later
// segment its initial state; then those segments run again with outputs, all
// in parallel.
constexpr int kSegOut = 0;   // outputs; state from h0 (NULL: zero), final to hT
constexpr int kSegBoth = 1;  // no outputs; R (from zero) to hT and P to hP
constexpr int kMaxSegItems = 64;
constexpr int kPhasePrep = 1;   // launch the prep kernel
constexpr int kPhaseState = 2;  // launch the state pass

struct SegItem {
  int r, c0, c1, mode;  // sequence r, its chunks [c0, c1)
  int pool_h0, pool_hT; // nonzero: the state at the sequence's pool row (kernel arguments h0 / hT)
  const float* h0;      // else [Hv, D, D] initial state of the item (NULL: zero)
  float* hT;            // else [Hv, D, D] final state (NULL: not stored)
  float* hP;            // kSegBoth: [Hv, D, D] the segment's transition P
};
struct SegList {
  int n = 0;  // 0: one item per sequence, states at the pool rows (the plain launch)
  int n_narrow = 0;  // items 0 .. n_narrow - 1 run in 32-column workgroups (the rest in 64)
  SegItem it[kMaxSegItems];
};

template <int N>
struct NcTag {
  static constexpr int value = N;
};

// The recurrence of one 32-column tile of the state (ct: the tile within the
// workgroup's 64 columns, vc0 its first column), one workgroup barrier per
// chunk, from the identity's columns (ident), from ih0 or from zero; the final
// state goes to ihT.  kP: the transition of a segment -- U = 0 and nothing
// handed to the output waves (their exchange belongs to the chain waves of the
// same workgroup, which run the segment's own recurrence beside it).
template <int D, bool kP>
__device__ __forceinline__ void chain_pass(StateSmem<D>& sm, int ct, int vc0, int64_t nch, bool ident,
                                           const float* ih0, float* ihT, int h, int lane) {
  constexpr int NR = D / 32;
  constexpr int KS = D / 16;
  const int li = lane & 31, g = lane >> 5;
  f32x16_t S[NR];
  if (ident) {
    // the identity's columns vc0 + li (row position p holds key qswap(p))
#pragma unroll
    for (int rt = 0; rt < NR; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          S[rt][4 * i + rr] = qswap(32 * rt + 8 * i + 4 * g + rr) == vc0 + li ? 1.f : 0.f;
  } else if (ih0) {
    const float* hp = ih0 + static_cast<int64_t>(h) * D * D + vc0 + li;
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
    StateXchgV& X = sm.xv[jc & 1];
    (void)X;
    // Re-derive lane indices from an opaque copy each chunk so the compiler
    // does not keep every lane-dependent address live across the loop.
    int tid_l = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid_l));
    const int ln = tid_l & 63;

    // Operand fragments of each product are read from LDS as one batch ahead
    // of its MFMAs, so the reads overlap each other instead of each MFMA
    // waiting out an LDS latency: first the V^T and T'' fragments of
    // U = T'' V (the products -W S accumulate onto; U = 0 for a transition),
    // then -W in k-step order.
    f32x16_t U[2] = {zero16(), zero16()};
    h16x8_t wf[2][KS];
    s16x8_t vcf[2][2];
    h16x8_t tbf[6];
    if constexpr (!kP) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int h = 0; h < 2; ++h) vcf[tt][h] = B.Vc[ct][tt][h][ln];
#pragma unroll
      for (int j = 0; j < 6; ++j) tbf[j] = B.Tb[j][ln];
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      wf[0][s] = B.W[s][ln];
      wf[1][s] = B.W[KS + s][ln];
    }
    const float eg = B.vec[2 * kC];
    __builtin_amdgcn_sched_barrier(0);
    // S as fp16 fragments (B operand of W S here, A operand of the output
    // wave's S^T Q'^T), packed while the reads are in flight.  Vn = U + (-W) S
    // with both 32-token tiles interleaved; tile 1's last product is issued
    // after the fence below, so tile 0 is packed while it runs.
    h16x8_t Sh[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) Sh[s] = (s & 1) ? pack_h8<8>(S[s >> 1]) : pack_h8<0>(S[s >> 1]);
    // the exchange copy of S goes out at once (its flag follows the products,
    // by when the writes have landed), and the decay of the old state sits
    // between the products: nothing in this region waits on them
    if constexpr (!kP) {
#pragma unroll
      for (int s = 0; s < KS; ++s) sm.xs.Sh[ct][s][ln] = Sh[s];
      // V^T by the natural identity (exact), then U = T'' V: these products
      // do not wait on S, and the decay below runs while they do (the same
      // products in the same order as a separate wave's would be)
      const s16x8_t in0 = ident_frag(0, ln & 31, ln >> 5), in1 = ident_frag(1, ln & 31, ln >> 5);
      f32x16_t vt[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        vt[tt] = mfma32_bf16(vcf[tt][0], in0, zero16());
        vt[tt] = mfma32_bf16(vcf[tt][1], in1, vt[tt]);
      }
      h16x8_t vbf[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) vbf[ks] = (ks & 1) ? pack_h8<8>(vt[ks >> 1]) : pack_h8<0>(vt[ks >> 1]);
      U[0] = mfma32(tbf[0], vbf[0], U[0]);
      U[1] = mfma32(tbf[2], vbf[0], U[1]);
      U[0] = mfma32(tbf[1], vbf[1], U[0]);
      U[1] = mfma32(tbf[3], vbf[1], U[1]);
      U[1] = mfma32(tbf[4], vbf[2], U[1]);
      U[1] = mfma32(tbf[5], vbf[3], U[1]);
    }
#pragma unroll
    for (int rt = 0; rt < NR; ++rt)
#pragma unroll
      for (int e = 0; e < 16; ++e) S[rt][e] *= eg;
#pragma unroll
    for (int s = 0; s < KS - 1; ++s) {
      U[0] = mfma32(wf[0][s], Sh[s], U[0]);
      U[1] = mfma32(wf[1][s], Sh[s], U[1]);
    }
    U[0] = mfma32(wf[0][KS - 1], Sh[KS - 1], U[0]);
    // the flag that says S is in the exchange: every lane stores the count to
    // its own word (no branch, so the region above stays one schedule); the
    // output waves read word 0
    if constexpr (!kP) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
      __hip_atomic_store(&sm.sflag[ct][ln], static_cast<int>(jc) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    h16x8_t kf[NR][4];
#pragma unroll
    for (int rt = 0; rt < NR; ++rt)
#pragma unroll
      for (int s = 0; s < 4; ++s) kf[rt][s] = B.Kt[rt * 4 + s][ln];
    // cK of the tokens 32 mt + 8 i + 4 lgp + r held by this lane's Vn elements
    f32x4_t ck[2][4];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        ck[mt][i] = *reinterpret_cast<const f32x4_t*>(&B.vec[kC + 32 * mt + 8 * i + 4 * (ln >> 5)]);
    __builtin_amdgcn_sched_barrier(0);
    U[1] = mfma32(wf[1][KS - 1], Sh[KS - 1], U[1]);
    // S <- e^gamma S + K^T diag(cK) Vn, one token tile at a time: Vn as fp16
    // (A operand of Vn^T A^T, to the exchange) and diag(cK) Vn as fp16 (B
    // operand of the update); tile 1 is packed while tile 0's products run.
    // The exchange gets Vn as its fp16 rounding Vh and the rounding's
    // residual Vl, formed while the update's products run.
    h16x8_t Vh[4], Vk[4];
    f32x16_t Uk[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      Vh[2 * mt] = pack_h8<0>(U[mt]);
      Vh[2 * mt + 1] = pack_h8<8>(U[mt]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) Uk[mt][4 * i + r] = U[mt][4 * i + r] * ck[mt][i][r];
      Vk[2 * mt] = pack_h8<0>(Uk[mt]);
      Vk[2 * mt + 1] = pack_h8<8>(Uk[mt]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 2 * mt; s < 2 * mt + 2; ++s)
#pragma unroll
        for (int rt = 0; rt < NR; ++rt) S[rt] = mfma32(kf[rt][s], Vk[s], S[rt]);
    }
    if constexpr (!kP) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const u32x4_t hi = __builtin_bit_cast(u32x4_t, Vh[s]);
        u32x4_t lo;
#pragma unroll
        for (int p2 = 0; p2 < 4; ++p2) {
          const int e = 8 * (s & 1) + 2 * p2;
          lo[p2] = f2h2_lo(U[s >> 1][e], U[s >> 1][e + 1], hi[p2]);
        }
        X.Vh[ct][s][ln] = Vh[s];
        X.Vl[ct][s][ln] = __builtin_bit_cast(h16x8_t, lo);
      }
    }
    gdn::lds_barrier();
  }

  if (ihT) {
    // lane indices re-derived here, so none of the loop's is kept live across it
    int tid_l = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid_l));
    const int le = tid_l & 31, ge = (tid_l >> 5) & 1;
    float* hp = ihT + static_cast<int64_t>(h) * D * D + vc0 + le;
#pragma unroll
    for (int rt = 0; rt < NR; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          hp[static_cast<int64_t>(qswap(32 * rt + 8 * i + 4 * ge + rr)) * D] = S[rt][4 * i + rr];
  }
}



// grid = state_grid(...) (the 32-column region, then the 64-column one); block = 64 * 8.
// Workgroup (item: sequence r or a segment of it, value head h, column block cb) owns state columns
// col0 .. col0 + 32 nc - 1 (nc = 2 tiles of 32, or 1 in the 32-column region; col0 = 32 nc cb).
// kMix: the instance that holds the 32-column paths (launched only when the item list has
// 32-column items).  One workgroup barrier per chunk j: before it the
// chain consumes stage j % 2 and writes exchange j % 2, the K and U waves fill
// stage (j + 1) % 2, and the output waves read exchange (j - 1) % 2.  No wave
// reads what another wave wrote before the barrier that separates them.
template <int D, bool kX, bool kMix>
__global__ __launch_bounds__(64 * kStateWaves) void chunk_state_kernel(
    const uint16_t* __restrict__ v, int64_t sv, const uint8_t* __restrict__ ws, const float* h0, float* hT,
    const int64_t* __restrict__ ids, int64_t sstride, const int64_t* __restrict__ cu, int n_seqs, int Hv,
    uint16_t* __restrict__ o, StateConv cr, const uint8_t* __restrict__ fresh, SegList segs) {
  constexpr int NR = D / 32;  // 32-row tiles of the state
  constexpr int KS = D / 16;  // k-steps over keys
  __shared__ StateSmem<D> sm;
  __shared__ long long s_base;

  // Work item wi = (item * Hv + h) * ncb + cb within a region.  The (item, head) pairs go
  // round-robin over the 8 XCDs (workgroup b runs on XCD b % 8), so every
  // sequence's heads spread over all XCDs and a long sequence does not leave
  // its XCD's L2 and fabric link loaded while others idle; the ncb column
  // blocks of a head are consecutive on one XCD and share its record reads
  // in that XCD's L2.  A region has 8 * ceil(items * Hv / 8) * ncb workgroups.
  // Two grid regions: the first n_narrow items in 32-column workgroups (one
  // chain, nc = 1 tile of 32 columns, D / 32 blocks per head), then the rest
  // in 64-column ones (nc = 2).  The first region is a multiple of 8
  // workgroups, so workgroup b runs on XCD b % 8 in both.
  const int64_t n_items = segs.n ? segs.n : n_seqs;
  // (kMix: the instance that holds the 32-column paths; the 64-column-only
  // instance leaves them out, so its code is not shaped by them)
  const int64_t n_nar = kMix && segs.n ? segs.n_narrow : 0;
  const int64_t grid_nar =
      n_nar ? gdn::kNumXcd * ((n_nar * Hv + gdn::kNumXcd - 1) / gdn::kNumXcd) * (D / 32) : 0;
  const bool narrow = kMix && blockIdx.x < grid_nar;
  const int nc = narrow ? 1 : 2;  // 32-column state tiles of the workgroup
  const int ncb = D / (32 * nc);  // column blocks per head
  int64_t wi, item0;
  {
    const int64_t b = narrow ? blockIdx.x : blockIdx.x - grid_nar;
    item0 = narrow ? 0 : n_nar;
    const int64_t n_reg = narrow ? n_nar : n_items - n_nar;
    const int64_t xcd = b % gdn::kNumXcd, k = b / gdn::kNumXcd;
    const int64_t pair = (k / ncb) * gdn::kNumXcd + xcd;
    if (pair >= n_reg * Hv) return;
    wi = pair * ncb + k % ncb;
  }
  const int cb = static_cast<int>(wi % ncb);
  const int h = static_cast<int>((wi / ncb) % Hv);
  const int item = static_cast<int>(item0 + wi / (static_cast<int64_t>(ncb) * Hv));
  const int col0 = cb * 32 * nc;  // the workgroup's first state column
  int r, mode;
  int64_t c0;
  int64_t nch;  // chunks of the item
  const float* ih0;
  float* ihT;
  const int64_t seq_bos = segs.n ? cu[segs.it[item].r] : cu[item];
  const int64_t seq_len = (segs.n ? cu[segs.it[item].r + 1] : cu[item + 1]) - seq_bos;
  {
    int pool_h0 = 1, pool_hT = 1;
    if (segs.n) {
      const SegItem& it = segs.it[item];
      r = it.r;
      c0 = it.c0;
      nch = it.c1 - it.c0;
      mode = it.mode;
      pool_h0 = it.pool_h0;
      pool_hT = it.pool_hT;
      ih0 = it.h0;
      ihT = it.hT;
    } else {
      r = item;
      c0 = 0;
      nch = chunks_of(seq_len);
      mode = kSegOut;
    }
    const int64_t srow = ids ? ids[r] : r;
    if (pool_h0) ih0 = h0 && !(fresh && fresh[r]) ? h0 + srow * sstride : nullptr;
    if (pool_hT) ihT = hT ? hT + srow * sstride : nullptr;
  }
  // the item's tokens
  const int64_t bos = seq_bos + c0 * kC;
  const int64_t seqlen = min<int64_t>(seq_len - c0 * kC, nch * kC);

  // first workspace chunk of this sequence: sum of earlier sequences' chunks
  if (threadIdx.x < 64) {
    long long part = 0;
    for (int rr = threadIdx.x; rr < r; rr += 64) part += chunks_of(cu[rr + 1] - cu[rr]);
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) part += __shfl_xor(part, m, 64);
    if (threadIdx.x == 0) s_base = part;
  }
  if (threadIdx.x < 128) sm.sflag[threadIdx.x >> 6][threadIdx.x & 63] = 0;
  __syncthreads();
  const int64_t cbase = s_base + c0;
  const int64_t rec_stride = static_cast<int64_t>(Hv) * rec_bytes(D);
  const uint8_t* rec0 = ws + cbase * rec_stride + static_cast<int64_t>(h) * rec_bytes(D);

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int li = lane & 31, g = lane >> 5;
  // A narrow workgroup's second chain wave has no columns: it takes part in
  // the nch + 1 barriers every other wave takes.
  if (kMix && nc == 1 && wave == 1) {
    if (nch > 0)
      for (int64_t j = 0; j <= nch; ++j) gdn::lds_barrier();
    return;
  }

#define GDN_LEN(j_) static_cast<int>(min<int64_t>(kC, seqlen - (j_) * kC))
  if (wave >= 2) {
    // one item per sequence (its first chunk, with outputs) rolls the conv
    // state, in its output waves at the start of interval 0
    const bool roll = kX && wave < 4 && c0 == 0 && mode == kSegOut;
#define GDN_ROLL() \
  conv_roll<D>(cr, ids ? ids[r] : r, fresh && fresh[r], seq_bos, seq_len, h, col0, 32 * nc, threadIdx.x - 128, 128)
    if (nch == 0) {
      if (roll) GDN_ROLL();
      return;
    }
    if (wave < 4 && mode == kSegBoth) {
      // the segment's transition P on the output waves: the chain of column
      // tile wave - 2 from the identity's columns, with U = 0 (one barrier
      // before the first chunk and one per chunk, like every role)
      chain_pass<D, true>(sm, wave - 2, col0 + 32 * (wave - 2), nch, true, nullptr, segs.it[item].hP, h, lane);
      return;
    }
    // ------------------------------------------------------------ output --
    // (NC: the workgroup's 32-column tiles, a compile-time count for the
    // accumulators)
    auto output_role = [&](auto nc_tag, auto nt_tag) {
      constexpr int NC = decltype(nc_tag)::value;
      constexpr int NT = decltype(nt_tag)::value;  // the wave's token tile
      // In the interval of chunk c (between workgroup barriers c and c + 1)
      // an output wave finishes chunk c - 1 (Vn^T A^T, the store) and runs
      // S^T Q'^T of chunk c.  Chunk c's Q' fragments live in register set
      // c % 2 and its A fragments in set c % 2; each set is reloaded (for
      // chunk c + 2, resp. c + 1) as soon as it has been read, so a load has
      // more than an interval to arrive.  The compiler's load counters must
      // stay exact for that, so no load may look younger than it is: every
      // path issues the same loads (past the last chunk they repeat it), the
      // sets go out oldest first, and the loop has a single exit (two chunks
      // per trip, the odd one after it).  Each tile's role is compiled on its
      // own, so the A loads (two fragment pairs for tile 0, four for tile 1)
      // are exact on each path.
      constexpr int nt = NT;
      uint16_t* oh = o + (bos * Hv + h) * D + col0;
      const int64_t ostride = static_cast<int64_t>(kC) * Hv * D;
      QPrefetch<D> q0, q1;
      APrefetch a0, a1;
      f32x16_t acc[NC];
      const uint8_t* rec1 = rec0 + min<int64_t>(1, nch - 1) * rec_stride;
      q_prefetch<D>(q0, rec0, nt, lane);
      gdn::keep_loads_here();  // the sets go out oldest first, as in the loop
      a_prefetch<NT>(a0, rec0, lane);
      gdn::keep_loads_here();
      q_prefetch<D>(q1, rec1, nt, lane);
      gdn::keep_loads_here();
      a_prefetch<NT>(a1, rec1, lane);
      gdn::keep_loads_here();
      gdn::lds_barrier();
      // The conv-state roll, in interval 0: the U waves have read the old v
      // taps before the first barrier (and the prep kernel the q and k taps
      // before this kernel), and interval 0 has no finished chunk to store, so
      // the roll stays off the tail of the workgroups that finish last.
      if (roll) GDN_ROLL();
      // interval 0: S^T Q'^T of chunk 0
      o_inter<D, NC>(q0, rec0 + min<int64_t>(2, nch - 1) * rec_stride, sm.xs, &sm.sflag[0][0], 0, nt, lane, acc);
      gdn::keep_loads_here();
      gdn::lds_barrier();
#define GDN_OITER(jj, QC, AP)                                                                               \
  o_intra<NC, NT>(AP, sm.xv[((jj) - 1) & 1], acc, lane);                                                   \
  __builtin_amdgcn_sched_barrier(0);                                                                        \
  a_prefetch<NT>(AP, rec0 + min<int64_t>((jj) + 1, nch - 1) * rec_stride, lane);                            \
  gdn::keep_loads_here();                                                                                   \
  o_store<NC>(acc, sm.ot[nt], oh + ((jj) - 1) * ostride, kC, Hv, D, nt, lane);                              \
  o_inter<D, NC>(QC, rec0 + min<int64_t>((jj) + 2, nch - 1) * rec_stride, sm.xs, &sm.sflag[0][0], jj, nt, lane, \
                 acc);                                                                                      \
  gdn::keep_loads_here();                                                                                   \
  gdn::lds_barrier();
      int64_t j = 1;
      for (; j + 1 < nch; j += 2) {
        GDN_OITER(j, q1, a0)      // finishes chunk j - 1 (even), starts chunk j (odd)
        GDN_OITER(j + 1, q0, a1)  // finishes chunk j (odd), starts chunk j + 1 (even)
      }
      if (j < nch) {
        GDN_OITER(j, q1, a0)
      }
#undef GDN_OITER
      if ((nch - 1) & 1)
        o_intra<NC, NT>(a1, sm.xv[1], acc, lane);
      else
        o_intra<NC, NT>(a0, sm.xv[0], acc, lane);
      o_store<NC>(acc, sm.ot[nt], oh + (nch - 1) * ostride, GDN_LEN(nch - 1), Hv, D, nt, lane);
    };
    if (wave < 4) {
      if ((!kMix || nc == 2) && wave == 2)
        output_role(NcTag<2>{}, NcTag<0>{});
      else if (!kMix || nc == 2)
        output_role(NcTag<2>{}, NcTag<1>{});
      else if (wave == 2)
        output_role(NcTag<1>{}, NcTag<0>{});
      else
        output_role(NcTag<1>{}, NcTag<1>{});
#undef GDN_ROLL
    } else {
      // ------------------------------------------------------------ U and K --
      // Chunk c's inputs live in register set c % 3; the loads of chunk j + 3
      // go out before chunk j + 1 is staged, two iterations ahead of their use.
      // The loop runs three chunks per trip so each set stays a fixed set of
      // registers; as for the output waves, every path issues the same loads,
      // oldest set first, and the loop has a single exit.
#define GDN_PITER(jj, LD, ST, PREFETCH, STAGE)               \
  PREFETCH(LD, min<int64_t>((jj) + 3, nch - 1));             \
  gdn::keep_loads_here();                                    \
  if ((jj) + 1 < nch) STAGE(ST, (jj) + 1);                   \
  gdn::lds_barrier();
      // U waves: in a 64-column workgroup wave 6 + c takes tile c (both of
      // its 16-column halves), in a 32-column one wave 6 + hb takes half hb of
      // the one tile (NH: halves per wave, a compile-time count; the wave's
      // halves sit in register slots 0 .. NH - 1, hb only moves addresses)
      auto u_role = [&](auto nh_tag) {
        constexpr int NH = decltype(nh_tag)::value;
        const int u = wave - 6;
        const int c = NH == 2 ? u : 0;
        const int hb = NH == 2 ? 0 : u;
        const uint16_t* vh = v + static_cast<int64_t>(h) * D + col0;
        const int svi = static_cast<int>(sv);
        // fused: the conv taps of the tile's channels into LDS, and the carry
        // rows of the first chunk's window (the rows before the item, or
        // before a sequence its state's taps -- zero, not read, when fresh)
        s16x8_t carry[2] = {s16x8_t{0, 0, 0, 0, 0, 0, 0, 0}, s16x8_t{0, 0, 0, 0, 0, 0, 0, 0}};
        if constexpr (kX) {
          const int li = lane & 31, g = lane >> 5;
          const int64_t ch0 = 2LL * cr.key_dim + static_cast<int64_t>(h) * D + col0 + 32 * c;
          if (lane < 32) {
            // channel ch0 + lane's 4 taps, as fp32
            const uint2 wb = reinterpret_cast<const uint2*>(cr.w + ch0 * 4)[lane];
            reinterpret_cast<float4*>(sm.vw[u])[lane] =
                make_float4(lo_half(wb.x), hi_half(wb.x), lo_half(wb.y), hi_half(wb.y));
          }
          const int64_t ch = ch0 + 8 * g;
          if (c0 != 0) {
            const uint16_t* hp = vh + (bos - 3 + min(li, 2)) * sv + 32 * c + 8 * g;
#pragma unroll
            for (int i = 0; i < NH; ++i) carry[i] = *reinterpret_cast<const s16x8_t*>(hp + 16 * (hb + i));
          } else if (!(fresh && fresh[r])) {
            const uint16_t* sp = cr.cstate + (ids ? ids[r] : r) * cr.ss_seq + ch * cr.ss_ch + min(li, 2);
#pragma unroll
            for (int i = 0; i < NH; ++i)
#pragma unroll
              for (int e = 0; e < 8; ++e) carry[i][e] = static_cast<short>(sp[(16 * (hb + i) + e) * cr.ss_ch]);
          }
          wave_sync();
        }
#define GDN_UPF(P, jc) u_prefetch<NH>(P, vh, svi, bos + (jc) * kC, GDN_LEN(jc), c, hb, lane)
#define GDN_UST(P, jc) u_stage<D, kX, NH>(P, sm.st[(jc) & 1], c, hb, lane, carry, sm.vtile[u], sm.vw[u])
        UPrefetch p0, p1, p2;
        GDN_UPF(p0, 0);
        gdn::keep_loads_here();  // the sets go out oldest first, as in the loop
        GDN_UPF(p1, min<int64_t>(1, nch - 1));
        gdn::keep_loads_here();
        GDN_UPF(p2, min<int64_t>(2, nch - 1));
        gdn::keep_loads_here();
        GDN_UST(p0, 0);
        gdn::lds_barrier();
        int64_t j = 0;
        for (; j + 2 < nch; j += 3) {
          GDN_PITER(j, p0, p1, GDN_UPF, GDN_UST)
          GDN_PITER(j + 1, p1, p2, GDN_UPF, GDN_UST)
          GDN_PITER(j + 2, p2, p0, GDN_UPF, GDN_UST)
        }
        if (j < nch) {
          GDN_PITER(j, p0, p1, GDN_UPF, GDN_UST)
        }
        if (j + 1 < nch) {
          GDN_PITER(j + 1, p1, p2, GDN_UPF, GDN_UST)
        }
#undef GDN_UPF
#undef GDN_UST
      };
      if (wave >= 6) {
        if (!kMix || nc == 2)
          u_role(NcTag<2>{});
        else
          u_role(NcTag<1>{});
      } else {
        // Chunk c's inputs live in register set c % 2; each stage issues the
        // loads of the chunk two ahead as soon as it has read the registers
        // they land in, so a load has two chunk steps to arrive.  As for the
        // other roles, every path issues the same loads, oldest set first, and
        // the loop (two chunks per trip) has a single exit.
        const int pk = wave - 4;
#define GDN_KSTAGE(P, jc, jn) k_stage<D>(P, sm.st[(jc) & 1], pk, lane, rec0 + (jn) * rec_stride)
        KPrefetch<D> p0, p1;
        k_prefetch_kt<D>(p0, rec0, pk, lane);
        k_prefetch_tw<D>(p0, rec0, pk, lane);
        gdn::keep_loads_here();
        k_prefetch_kt<D>(p1, rec0 + min<int64_t>(1, nch - 1) * rec_stride, pk, lane);
        k_prefetch_tw<D>(p1, rec0 + min<int64_t>(1, nch - 1) * rec_stride, pk, lane);
        gdn::keep_loads_here();
        GDN_KSTAGE(p0, 0, min<int64_t>(2, nch - 1));
        gdn::lds_barrier();
        int64_t j = 0;
        for (; j + 2 < nch; j += 2) {
          GDN_KSTAGE(p1, j + 1, min<int64_t>(j + 3, nch - 1));
          gdn::lds_barrier();
          GDN_KSTAGE(p0, j + 2, min<int64_t>(j + 4, nch - 1));
          gdn::lds_barrier();
        }
        if (j + 1 < nch) {
          GDN_KSTAGE(p1, j + 1, min<int64_t>(j + 3, nch - 1));
          gdn::lds_barrier();
        }
        gdn::lds_barrier();  // the last chunk: nothing left to stage
#undef GDN_KSTAGE
      }
#undef GDN_PITER
    }
    return;
  }
#undef GDN_LEN

  // -------------------------------------------------------------- chain --
  chain_pass<D, false>(sm, wave, col0 + 32 * wave, nch, false, ih0, ihT, h, lane);
}
// ---- segment scan ----
// For each split sequence: S_1 = the first segment's final state, then
// S_{s+1} = P_s S_s + R_s for its middle segments s = 1 .. m, in fp32 (the
// sum over keys in order).  States are [Hv, D, D] (row = key).
constexpr int kMaxSeg = 12;     // segments per sequence
constexpr int kMaxChains = 16;  // split sequences per call
struct ScanChain {
  float* S;        // [m + 1][Hv, D, D]: S_1 (read), S_2 .. S_{m+1} (written)
  const float* P;  // [m][Hv, D, D]: P_1 .. P_m
  const float* R;  // [m][Hv, D, D]: R_1 .. R_m
  int m;
};
struct ScanList {
  int n;
  ScanChain c[kMaxChains];
};

// grid = 8 * ceil(n_chains * Hv * D / 16 / 8), block = 256: workgroup (chain,
// head, 16 state columns); thread = one key row k and OPT consecutive columns.
// Each step is P_s (D x D) times the block of S_s (D x 16) in fp32 FMAs, the
// sum over keys in order.  P_s is staged in LDS with rows padded to D + 1
// floats (the threads' reads of their rows at one key hit distinct banks);
// P_s and R_s are loaded one step ahead and the barriers order LDS only, so
// those loads stay in flight across them (every step issues the same loads,
// the last one repeating itself).
// (D = 64; D = 128 runs seg_scan_mfma_kernel below)
template <int D>
__global__ __launch_bounds__(256) void seg_scan_kernel(ScanList sl, int Hv) {
  constexpr int CB = 16;
  constexpr int NB = D / CB;
  constexpr int OPT = D * CB / 256;    // outputs per thread: 4 at D = 64
  constexpr int TPR = CB / OPT;        // threads per row
  constexpr int PL = D + 1;            // padded row of P in LDS
  constexpr int NV = D * D / 4 / 256;  // float4 loads of P per thread
  __shared__ float Ps[D * PL];
  __shared__ __align__(16) float Ss[D][CB];
  // the column blocks of a head share one XCD, so its L2 fetches each P_s once
  const int64_t wi = gdn::xcd_remap(blockIdx.x, static_cast<int64_t>(sl.n) * Hv * NB);
  if (wi < 0) return;
  const int blk = static_cast<int>(wi % NB);
  const int h = static_cast<int>((wi / NB) % Hv);
  const int ci = static_cast<int>(wi / (NB * Hv));
  const ScanChain& c = sl.c[ci];
  const int64_t hs = static_cast<int64_t>(Hv) * D * D;  // one state
  const int64_t hp = static_cast<int64_t>(h) * D * D;
  const int k = threadIdx.x / TPR, col = (threadIdx.x % TPR) * OPT;
  const int64_t off = hp + static_cast<int64_t>(k) * D + blk * CB + col;
#pragma unroll
  for (int o = 0; o < OPT; ++o) Ss[k][col + o] = c.S[off + o];
  float4 pre[NV];
  float rpre[OPT];
  auto prefetch = [&](int st) {
    const float4* pg = reinterpret_cast<const float4*>(c.P + st * hs + hp);
#pragma unroll
    for (int i = 0; i < NV; ++i) pre[i] = pg[threadIdx.x + 256 * i];
#pragma unroll
    for (int o = 0; o < OPT; ++o) rpre[o] = c.R[st * hs + off + o];
  };
  prefetch(0);
  gdn::keep_loads_here();
  for (int s = 0; s < c.m; ++s) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int e = 4 * (threadIdx.x + 256 * i);
      float* dst = &Ps[(e / D) * PL + e % D];
      dst[0] = pre[i].x;
      dst[1] = pre[i].y;
      dst[2] = pre[i].z;
      dst[3] = pre[i].w;
    }
    float acc[OPT];
#pragma unroll
    for (int o = 0; o < OPT; ++o) acc[o] = rpre[o];
    gdn::lds_barrier();  // P_s and S_s are in LDS
    prefetch(min(s + 1, c.m - 1));
    gdn::keep_loads_here();
#pragma unroll 8
    for (int m = 0; m < D; ++m) {
      const float pv = Ps[k * PL + m];
#pragma unroll
      for (int o4 = 0; o4 < OPT / 4; ++o4) {
        const float4 sv = *reinterpret_cast<const float4*>(&Ss[m][col + 4 * o4]);
        acc[4 * o4] = fmaf(pv, sv.x, acc[4 * o4]);
        acc[4 * o4 + 1] = fmaf(pv, sv.y, acc[4 * o4 + 1]);
        acc[4 * o4 + 2] = fmaf(pv, sv.z, acc[4 * o4 + 2]);
        acc[4 * o4 + 3] = fmaf(pv, sv.w, acc[4 * o4 + 3]);
      }
    }
    gdn::lds_barrier();  // every row of S_s and P_s is read
#pragma unroll
    for (int o = 0; o < OPT; ++o) {
      Ss[k][col + o] = acc[o];
      c.S[(s + 1) * hs + off + o] = acc[o];
    }
  }
}

// The scan at D = 128 on the fp32 matrix cores: workgroup (chain, head, 16
// state columns); wave w computes rows 32 w .. 32 w + 31 of
// S_{s+1}[:, block] = P_s S_s[:, block] + R_s[:, block] as two 16 x 16 tiles
// of v_mfma_f32_16x16x4_f32 over the 32 key steps (lane (c, g) holds A
// element (row c, key 4 kk + g), B element (key 4 kk + g, column c), C rows
// 4 g + i of column c).  P_s goes through LDS once per step (row pitch D + 4
// floats: the 64 lanes of an A read hit distinct banks); S_s is re-staged in
// LDS between steps; P_s and R_s are loaded one step ahead, as in the VALU
// form above.  (Config 3's scan: 45 us in the VALU form at D = 128.)
__global__ __launch_bounds__(256) void seg_scan_mfma_kernel(ScanList sl, int Hv) {
  constexpr int D = 128;
  constexpr int CB = 16;
  constexpr int NB = D / CB;
  constexpr int PL = D + 4;
  constexpr int NV = D * D / 4 / 256;  // float4 loads of P per thread
  __shared__ __align__(16) float Ps[D * PL];
  __shared__ __align__(16) float Ss[D][CB];
  const int64_t wi = gdn::xcd_remap(blockIdx.x, static_cast<int64_t>(sl.n) * Hv * NB);
  if (wi < 0) return;
  const int blk = static_cast<int>(wi % NB);
  const int h = static_cast<int>((wi / NB) % Hv);
  const int ci = static_cast<int>(wi / (NB * Hv));
  const ScanChain& c = sl.c[ci];
  const int64_t hs = static_cast<int64_t>(Hv) * D * D;
  const int64_t hp = static_cast<int64_t>(h) * D * D;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int lc = lane & 15, lg = lane >> 4;
  for (int e = tid; e < D * CB; e += 256) Ss[e / CB][e % CB] = c.S[hp + static_cast<int64_t>(e / CB) * D + blk * CB + e % CB];
  // the lane's C elements: rows r0 + 16 t + i, column lc
  const int r0 = 32 * wave + 4 * lg;
  const int64_t coff = hp + static_cast<int64_t>(r0) * D + blk * CB + lc;
  // P_s as float4 per thread (row-major: float4 f = tid + 256 i is row f / 32,
  // columns 4 (f % 32) ..) and the lane's 8 elements of R_s, one step ahead
  const f32x4_t* pg = reinterpret_cast<const f32x4_t*>(c.P + hp) + tid;
  const float* rg = c.R + coff;
  f32x4_t pre[NV];
  float rpre[8];
#pragma unroll
  for (int i = 0; i < NV; ++i) pre[i] = pg[256 * i];
#pragma unroll
  for (int j = 0; j < 8; ++j) rpre[j] = rg[static_cast<int64_t>(16 * (j >> 2) + (j & 3)) * D];
  gdn::keep_loads_here();
  for (int s = 0; s < c.m; ++s) {
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int f = tid + 256 * i;
      *reinterpret_cast<f32x4_t*>(&Ps[(f >> 5) * PL + 4 * (f & 31)]) = pre[i];
    }
    f32x4_t acc0 = {rpre[0], rpre[1], rpre[2], rpre[3]};
    f32x4_t acc1 = {rpre[4], rpre[5], rpre[6], rpre[7]};
    gdn::lds_barrier();  // P_s and S_s are in LDS
    const int64_t nx = static_cast<int64_t>(min(s + 1, c.m - 1)) * hs;
#pragma unroll
    for (int i = 0; i < NV; ++i) pre[i] = pg[nx / 4 + 256 * i];
#pragma unroll
    for (int j = 0; j < 8; ++j) rpre[j] = rg[nx + static_cast<int64_t>(16 * (j >> 2) + (j & 3)) * D];
    gdn::keep_loads_here();
    const float* pa = &Ps[(32 * wave + lc) * PL + lg];
#pragma unroll 8
    for (int kk = 0; kk < D / 4; ++kk) {
      const float bv = Ss[4 * kk + lg][lc];
      acc0 = gdn::mfma16x16x4f32(pa[4 * kk], bv, acc0);
      acc1 = gdn::mfma16x16x4f32(pa[16 * PL + 4 * kk], bv, acc1);
    }
    gdn::lds_barrier();  // every row of S_s and P_s is read
    float* so = c.S + (s + 1) * hs + coff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      Ss[r0 + i][lc] = acc0[i];
      Ss[r0 + 16 + i][lc] = acc1[i];
      so[static_cast<int64_t>(i) * D] = acc0[i];
      so[static_cast<int64_t>(16 + i) * D] = acc1[i];
    }
  }
}

// Segment plan of one call: how many segments each sequence is cut into.
// Only when few workgroups would run otherwise (n_seqs * Hv * D / 64 < 128) and
// the host knows the lengths.  max_segments: 0 = automatic (segments of at
// least 16 chunks, at most one workgroup per CU in the second pass), 1 =
// never, k >= 2 = up to k segments per sequence.
inline bool seg_eligible(int n_seqs, int Hv, int D) { return static_cast<int64_t>(n_seqs) * Hv * (D / kCB) < 128; }

// scratch bytes for the segment states of one call (an upper bound)
inline int64_t seg_scratch_bytes(int n_seqs, int Hv, int D) {
  if (!seg_eligible(n_seqs, Hv, D)) return 0;
  return static_cast<int64_t>(n_seqs) * (3 * kMaxSeg - 5) * Hv * D * D * 4;
}

struct SegPlan {
  int nseg[kMaxChains * 4];  // per sequence (<= 3 sequences eligible at Hv = 16)
  int len[kMaxChains * 4];   // chunks per segment
  bool any = false;
};

// (over the sequences selected by select_host, all if NULL)
inline SegPlan plan_segments(const int64_t* cu_host, const uint8_t* select_host, int n_seqs, int Hv, int D,
                             int max_segments, bool have_scratch) {
  SegPlan pl;
  int n_sel = 0;
  for (int r = 0; r < n_seqs; ++r) n_sel += !select_host || select_host[r];
  if (!cu_host || !have_scratch || max_segments == 1 || !seg_eligible(n_sel, Hv, D) || n_seqs > kMaxChains * 4)
    return pl;
  const int per_item = Hv * (D / kCB);
  int pass1 = 0, pass3 = 0, chains = 0;
  for (int r = 0; r < n_seqs; ++r) {
    pl.nseg[r] = 1;
    pl.len[r] = 1;
    if (select_host && !select_host[r]) continue;
    const int64_t nch = (cu_host[r + 1] - cu_host[r] + kC - 1) / kC;
    int S = 1;
    if (max_segments >= 2) {
      S = static_cast<int>(std::min<int64_t>(std::min(max_segments, kMaxSeg), nch));
    } else if (nch >= 32) {
      S = static_cast<int>(std::min<int64_t>(std::min(kMaxSeg, 256 / (per_item * n_sel) + 1), nch / 16));
    }
    int L = 1;
    if (S >= 2) {
      L = static_cast<int>((nch + S - 1) / S);
      S = static_cast<int>((nch + L - 1) / L);  // no empty last segment
    }
    if (S >= 2 && (chains + (S >= 3) > kMaxChains || pass1 + S - 1 > kMaxSegItems ||
                   pass3 + S - 1 > kMaxSegItems))
      S = 1;
    if (S < 2) {
      S = 1;
      pass1 += 1;
    } else {
      pass1 += S - 1;
      pass3 += S - 1;
      chains += S >= 3;
      pl.any = true;
    }
    if (pass1 > kMaxSegItems) return SegPlan{};
    pl.nseg[r] = S;
    pl.len[r] = L;
  }
  return pl;
}

// Column split of the plain state launch (gdn_set_column_split): 0 = by the
// estimate below, 1 = every sequence in 64-column workgroups, 2 = every
// sequence in 32-column ones.
int g_column_split = 0;

// Chunk period of a 32-column state workgroup, in 64-column periods: its output
// waves run one accumulation chain instead of two, and its single chain and U
// waves no longer share their SIMDs' issue with a second output tile.
constexpr double kNarrowPeriod = 0.93;

// Grid of the state launch: the narrow region (first n_narrow items, D / 32
// workgroups per head), then the wide one (D / 64 per head), each padded to a
// multiple of 8 workgroups as the kernel's mapping expects.
inline int64_t state_grid(int64_t items, int64_t n_narrow, int Hv, int D) {
  auto region = [&](int64_t n, int ncb) {
    return n ? gdn::kNumXcd * ((n * Hv + gdn::kNumXcd - 1) / gdn::kNumXcd) * ncb : 0;
  };
  return region(n_narrow, D / 32) + region(items - n_narrow, D / kCB);
}

// The plain launch's item list (no segments): the sequences longest first
// (longest-processing-time order, ties in sequence order), the k longest in
// 32-column workgroups.  A state workgroup fills its CU, so the pass is a list
// schedule of workgroups over the CUs in grid order, each taking nch chunk
// periods; k is the count (up to 4) whose estimated finish is lowest, narrow
// only where it saves at least 2 %.  Beyond two rounds of 64-column
// workgroups the estimate is skipped (k = 0): narrow ones only add to a full
// GPU there.  n = 0: the plain order does as well (no narrow item, and every
// workgroup starts at once).
inline SegList plan_columns(const int64_t* cu_host, int n_seqs, int Hv, int D) {
  SegList pl;
  if (!cu_host || n_seqs > kMaxSegItems || D % 64) return pl;
  int order[kMaxSegItems];
  int64_t nch[kMaxSegItems];
  for (int r = 0; r < n_seqs; ++r) {
    nch[r] = (cu_host[r + 1] - cu_host[r] + kC - 1) / kC;
    int i = r;
    for (; i > 0 && nch[order[i - 1]] < nch[r]; --i) order[i] = order[i - 1];
    order[i] = r;
  }
  const int wide_wgs = Hv * (D / kCB), nar_wgs = Hv * (D / 32);
  double ft[gdn::kNumCu];  // min-heap of the CUs' finish times
  auto finish = [&](int k) {
    int used = 0;
    double end = 0;
    for (int i = 0; i < n_seqs; ++i) {
      const bool nar = i < k;
      const double dur = static_cast<double>(nch[order[i]]) * (nar ? kNarrowPeriod : 1.0);
      const int m = nar ? nar_wgs : wide_wgs;
      for (int w = 0; w < m; ++w) {
        double t0 = 0;
        if (used < gdn::kNumCu) {
          ft[used++] = dur;
          std::push_heap(ft, ft + used, std::greater<double>());
        } else {
          std::pop_heap(ft, ft + used, std::greater<double>());
          t0 = ft[used - 1];
          ft[used - 1] = t0 + dur;
          std::push_heap(ft, ft + used, std::greater<double>());
        }
        end = std::max(end, t0 + dur);
      }
    }
    return end;
  };
  int k = 0;
  if (g_column_split == 2) {
    k = n_seqs;
  } else if (g_column_split == 0 && static_cast<int64_t>(n_seqs) * wide_wgs <= 2 * gdn::kNumCu) {
    double best = finish(0);
    for (int kk = 1; kk <= std::min(n_seqs, 4); ++kk) {
      const double t = finish(kk);
      if (t < 0.98 * best) {
        best = t;
        k = kk;
      }
    }
  }
  if (k == 0 && static_cast<int64_t>(n_seqs) * wide_wgs <= gdn::kNumCu) return pl;
  for (int i = 0; i < n_seqs; ++i) {
    SegItem& it = pl.it[pl.n++];
    it.r = order[i];
    it.c0 = 0;
    it.c1 = static_cast<int>(nch[order[i]]);
    it.mode = kSegOut;
    it.pool_h0 = 1;
    it.pool_hT = 1;
    it.h0 = nullptr;
    it.hT = nullptr;
    it.hP = nullptr;
  }
  pl.n_narrow = k;
  return pl;
}

template <int D>
int launch_chunk(const uint16_t* q, int64_t sq, const uint16_t* k, int64_t sk, const uint16_t* v,
                 int64_t sv, const float* g, const uint16_t* beta, const float* h0, float* hT,
                 const int64_t* ids, int64_t sstride, const int64_t* cu, const int64_t* cu_host, int max_segments,
                 int n_seqs, int64_t nc_bound, int Hk, int Hv, float scale, int l2norm, uint16_t* o, uint8_t* ws,
                 uint8_t* seg_ws, const ConvIn* cv, int phase, const uint8_t* select_host, hipStream_t stream) {
  // prep: one workgroup per (chunk, key head) when each key head has two value
  // heads, else per (chunk, value head)
  const int kR = Hv == 2 * Hk ? 2 : 1;
  const int64_t lwork = nc_bound * (Hv / kR);
  const int64_t lgrid = gdn::kNumXcd * ((lwork + gdn::kNumXcd - 1) / gdn::kNumXcd);
  StateConv cr{};
  if (cv)
    cr = StateConv{cv->x, cv->sx, const_cast<uint16_t*>(cv->cstate), cv->ss_seq, cv->ss_ch, cv->w, cv->key_dim, Hv / Hk};
  int st = GDN_OK;
  if (phase & kPhasePrep) {
    const dim3 pg(static_cast<unsigned>(lgrid)), pb(256);
    if (cv && kR == 2)
      chunk_prep_kernel<D, true, 2><<<pg, pb, 0, stream>>>(q, sq, k, sk, g, beta, cu, n_seqs, nc_bound, Hk, Hv, scale,
                                                           l2norm, ws, *cv);
    else if (cv)
      chunk_prep_kernel<D, true, 1><<<pg, pb, 0, stream>>>(q, sq, k, sk, g, beta, cu, n_seqs, nc_bound, Hk, Hv, scale,
                                                           l2norm, ws, *cv);
    else if (kR == 2)
      chunk_prep_kernel<D, false, 2><<<pg, pb, 0, stream>>>(q, sq, k, sk, g, beta, cu, n_seqs, nc_bound, Hk, Hv,
                                                            scale, l2norm, ws, ConvIn{});
    else
      chunk_prep_kernel<D, false, 1><<<pg, pb, 0, stream>>>(q, sq, k, sk, g, beta, cu, n_seqs, nc_bound, Hk, Hv,
                                                            scale, l2norm, ws, ConvIn{});
    st = gdn_launch_status();
    if (st != GDN_OK) return st;
  }
  if (!(phase & kPhaseState)) return GDN_OK;
  const uint8_t* fresh = cv ? cv->fresh : nullptr;
  auto state_launch = [&](const SegList& sl, int64_t items) {
    const int64_t n_nar = sl.n ? sl.n_narrow : 0;
    const int64_t cgrid = state_grid(items, n_nar, Hv, D);
    const dim3 gr(static_cast<unsigned>(cgrid)), bl(64 * kStateWaves);
    if (cv && n_nar)
      chunk_state_kernel<D, true, true><<<gr, bl, 0, stream>>>(v, sv, ws, h0, hT, ids, sstride, cu, n_seqs, Hv, o, cr,
                                                               fresh, sl);
    else if (cv)
      chunk_state_kernel<D, true, false><<<gr, bl, 0, stream>>>(v, sv, ws, h0, hT, ids, sstride, cu, n_seqs, Hv, o,
                                                                cr, fresh, sl);
    else if (n_nar)
      chunk_state_kernel<D, false, true><<<gr, bl, 0, stream>>>(v, sv, ws, h0, hT, ids, sstride, cu, n_seqs, Hv, o,
                                                                cr, fresh, sl);
    else
      chunk_state_kernel<D, false, false><<<gr, bl, 0, stream>>>(v, sv, ws, h0, hT, ids, sstride, cu, n_seqs, Hv, o,
                                                                 cr, fresh, sl);
    return gdn_launch_status();
  };
  auto item = [](int r, int64_t a, int64_t b, int mode, int ph0, int phT, const float* i0, float* iT,
                 float* iP = nullptr) {
    SegItem it;
    it.r = r;
    it.c0 = static_cast<int>(a);
    it.c1 = static_cast<int>(b);
    it.mode = mode;
    it.pool_h0 = ph0;
    it.pool_hT = phT;
    it.h0 = i0;
    it.hT = iT;
    it.hP = iP;
    return it;
  };
  const SegPlan pl = plan_segments(cu_host, select_host, n_seqs, Hv, D, max_segments, seg_ws != nullptr);
  if (!pl.any && !select_host) {
    const SegList plan = plan_columns(cu_host, n_seqs, Hv, D);
    if (plan.n) return state_launch(plan, plan.n);
    SegList none;
    none.n = 0;
    return state_launch(none, n_seqs);
  }
  // segment states: per split sequence S_1 .. S_{m+1}, P_1 .. P_m, R_1 .. R_m
  const int64_t hs = static_cast<int64_t>(Hv) * D * D;
  float* scratch = reinterpret_cast<float*>(seg_ws);
  SegList p1, p3;
  p1.n = 0;
  p3.n = 0;
  ScanList sc;
  sc.n = 0;
  for (int r = 0; r < n_seqs; ++r) {
    if (select_host && !select_host[r]) continue;
    const int S = pl.any ? pl.nseg[r] : 1;
    const int64_t L = pl.any ? pl.len[r] : 1;
    const int64_t nch = (cu_host[r + 1] - cu_host[r] + kC - 1) / kC;
    if (S < 2) {
      p1.it[p1.n++] = item(r, 0, nch, kSegOut, 1, 1, nullptr, nullptr);
      continue;
    }
    const int m = S - 2;
    float* Sst = scratch;  // S_1 .. S_{m+1}
    float* P = Sst + (m + 1) * hs;
    float* R = P + m * hs;
    scratch = R + m * hs;
    p1.it[p1.n++] = item(r, 0, L, kSegOut, 1, 0, nullptr, Sst);
    for (int s = 1; s <= m; ++s)
      p1.it[p1.n++] = item(r, s * L, (s + 1) * L, kSegBoth, 0, 0, nullptr, R + (s - 1) * hs, P + (s - 1) * hs);
    for (int s = 1; s < S; ++s)
      p3.it[p3.n++] = item(r, s * L, std::min<int64_t>((s + 1) * L, nch), kSegOut, 0, s == S - 1, Sst + (s - 1) * hs,
                           nullptr);
    if (m > 0) sc.c[sc.n++] = ScanChain{Sst, P, R, m};
  }
  if (p1.n == 0) return GDN_OK;
  st = state_launch(p1, p1.n);
  if (st != GDN_OK) return st;
  if (sc.n) {
    const int64_t swork = static_cast<int64_t>(sc.n) * Hv * (D / 16);
    const int64_t sgrid = gdn::kNumXcd * ((swork + gdn::kNumXcd - 1) / gdn::kNumXcd);
    if constexpr (D == 128)
      seg_scan_mfma_kernel<<<dim3(static_cast<unsigned>(sgrid)), dim3(256), 0, stream>>>(sc, Hv);
    else
      seg_scan_kernel<D><<<dim3(static_cast<unsigned>(sgrid)), dim3(256), 0, stream>>>(sc, Hv);
    st = gdn_launch_status();
    if (st != GDN_OK) return st;
  }
  return p3.n ? state_launch(p3, p3.n) : GDN_OK;
}

}  // namespace

// Column split of the plain state pass: 0 = by the list-schedule estimate
// (the default), 1 = every sequence in 64-column workgroups, 2 = every
// sequence in 32-column ones.  Process-wide; set it between calls.
extern "C" int gdn_set_column_split(int mode) {
  if (mode < 0 || mode > 2) return GDN_ERR_INVALID_ARG;
  g_column_split = mode;
  return GDN_OK;
}

extern "C" int64_t gdn_chunk_prefill_workspace_size(int64_t N, int n_seqs, int Hv, int D) {
  if (N < 0 || n_seqs < 0 || Hv <= 0 || (D != 64 && D != 128)) return -1;
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  return nc_bound * Hv * rec_bytes(D) + seg_scratch_bytes(n_seqs, Hv, D);
}

extern "C" int gdn_chunk_prefill(const uint16_t* q, int64_t sq_tok, const uint16_t* k,
                                 int64_t sk_tok, const uint16_t* v, int64_t sv_tok, const float* g,
                                 const uint16_t* beta, const float* h0, float* hT,
                                 const int64_t* state_ids, int64_t state_stride,
                                 const int64_t* cu_seqlens, const int64_t* cu_seqlens_host, int max_segments,
                                 int n_seqs, int64_t N, int Hk, int Hv,
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
  if (max_segments < 0) return GDN_ERR_INVALID_ARG;
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  if (workspace_bytes < gdn_chunk_prefill_workspace_size(N, n_seqs, Hv, D)) return GDN_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint8_t* seg_ws = seg_scratch_bytes(n_seqs, Hv, D) ? ws + nc_bound * Hv * rec_bytes(D) : nullptr;
  if (D == 128)
    return launch_chunk<128>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids, state_stride,
                             cu_seqlens, cu_seqlens_host, max_segments, n_seqs, nc_bound, Hk, Hv, scale, l2norm,
                             o, ws, seg_ws, nullptr, kPhasePrep | kPhaseState, nullptr, s);
  return launch_chunk<64>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids, state_stride,
                          cu_seqlens, cu_seqlens_host, max_segments, n_seqs, nc_bound, Hk, Hv, scale, l2norm, o,
                          ws, seg_ws, nullptr, kPhasePrep | kPhaseState, nullptr, s);
}

// workspace of the fused entry point: the same as the plain one's (the
// records, then the segment scratch)
extern "C" int64_t gdn_conv_chunk_prefill_workspace_size(int64_t N, int n_seqs, int Hv, int D) {
  return gdn_chunk_prefill_workspace_size(N, n_seqs, Hv, D);
}

// Argument checks of gdn_conv_chunk_prefill that do not depend on the
// workspace (shared with the allocation-free entry point).
static int conv_chunk_check(const uint16_t* x, int64_t sx_row, const uint16_t* conv_state, int64_t ss_seq,
                            int64_t ss_ch, const uint16_t* conv_w, const uint16_t* b, const uint16_t* a,
                            const void* A_log, const void* dt_bias, const float* h0, const float* hT,
                            int64_t state_stride, const int64_t* cu_seqlens, const int64_t* cu_seqlens_host,
                            int max_segments, int phase, const uint8_t* select_host, int n_seqs, int Hk, int Hv,
                            int D, const uint16_t* o) {
  if (!x || !conv_state || !conv_w || !a || !b || !A_log || !dt_bias || !cu_seqlens || !o)
    return GDN_ERR_INVALID_ARG;
  if (max_segments < 0 || phase < 1 || phase > 3) return GDN_ERR_INVALID_ARG;
  if (select_host && (!cu_seqlens_host || n_seqs > kMaxSegItems)) return GDN_ERR_INVALID_ARG;
  const int64_t C = 2LL * Hk * D + static_cast<int64_t>(Hv) * D;
  // 16-byte row segments of x, 8-byte output pieces
  if (sx_row % 8 || sx_row < C || sx_row >= (1LL << 24) || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(conv_w) % 16 || reinterpret_cast<uintptr_t>(o) % 8 || ss_ch < 3 ||
      ss_seq < C * ss_ch || ((h0 || hT) && state_stride < static_cast<int64_t>(Hv) * D * D))
    return GDN_ERR_INVALID_ARG;
  return GDN_OK;
}

// The launches of one checked call: records at ws, segment scratch at seg_ws
// (NULL: no segments).
static int conv_chunk_run(const uint16_t* x, int64_t sx_row, uint16_t* conv_state, int64_t ss_seq, int64_t ss_ch,
                          const uint16_t* conv_w, const uint16_t* b, const uint16_t* a, const void* A_log,
                          const void* dt_bias, int param_is_fp32, const float* h0, float* hT,
                          const int64_t* state_ids, const uint8_t* fresh, int64_t state_stride,
                          const int64_t* cu_seqlens, const int64_t* cu_seqlens_host, int max_segments, int phase,
                          const uint8_t* select_host, int n_seqs, int64_t N, int Hk, int Hv, int D, float scale,
                          int l2norm, uint16_t* o, uint8_t* ws, uint8_t* seg_ws, hipStream_t s) {
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  const ConvIn cv{x, sx_row, conv_state, ss_seq, ss_ch, state_ids, fresh, conv_w, Hk * D, a, b, A_log, dt_bias,
                  param_is_fp32 ? 1 : 0};
  // the state kernel's U waves read the raw v channels and run their conv
  const uint16_t* xv = x + 2LL * Hk * D;
  if (D == 128)
    return launch_chunk<128>(x, sx_row, x, sx_row, xv, sx_row, nullptr, nullptr, h0, hT, state_ids, state_stride,
                             cu_seqlens, cu_seqlens_host, max_segments, n_seqs, nc_bound, Hk, Hv, scale, l2norm,
                             o, ws, seg_ws, &cv, phase, select_host, s);
  return launch_chunk<64>(x, sx_row, x, sx_row, xv, sx_row, nullptr, nullptr, h0, hT, state_ids, state_stride,
                          cu_seqlens, cu_seqlens_host, max_segments, n_seqs, nc_bound, Hk, Hv, scale, l2norm, o,
                          ws, seg_ws, &cv, phase, select_host, s);
}

extern "C" int gdn_conv_chunk_prefill(const uint16_t* x, int64_t sx_row, uint16_t* conv_state,
                                      int64_t ss_seq, int64_t ss_ch, const uint16_t* conv_w,
                                      const uint16_t* b, const uint16_t* a, const void* A_log,
                                      const void* dt_bias, int param_is_fp32, const float* h0, float* hT,
                                      const int64_t* state_ids, const uint8_t* fresh, int64_t state_stride,
                                      const int64_t* cu_seqlens, const int64_t* cu_seqlens_host,
                                      int max_segments, int phase, const uint8_t* select_host, int n_seqs,
                                      int64_t N, int Hk, int Hv,
                                      int D, float scale, int l2norm, uint16_t* o, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (n_seqs < 0 || N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return GDN_ERR_INVALID_ARG;
  if (n_seqs == 0) return GDN_OK;
  const int st = conv_chunk_check(x, sx_row, conv_state, ss_seq, ss_ch, conv_w, b, a, A_log, dt_bias, h0, hT,
                                  state_stride, cu_seqlens, cu_seqlens_host, max_segments, phase, select_host,
                                  n_seqs, Hk, Hv, D, o);
  if (st != GDN_OK) return st;
  // 256-byte workspace records
  if (!workspace || reinterpret_cast<uintptr_t>(workspace) % 256) return GDN_ERR_INVALID_ARG;
  const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
  if (workspace_bytes < gdn_conv_chunk_prefill_workspace_size(N, n_seqs, Hv, D)) return GDN_ERR_INVALID_ARG;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint8_t* seg_ws = seg_scratch_bytes(n_seqs, Hv, D) ? ws + nc_bound * Hv * rec_bytes(D) : nullptr;
  return conv_chunk_run(x, sx_row, conv_state, ss_seq, ss_ch, conv_w, b, a, A_log, dt_bias, param_is_fp32, h0, hT,
                        state_ids, fresh, state_stride, cu_seqlens, cu_seqlens_host, max_segments, phase,
                        select_host, n_seqs, N, Hk, Hv, D, scale, l2norm, o, ws, seg_ws,
                        static_cast<hipStream_t>(stream));
}

// ---- the allocation-free variant of gdn_conv_chunk_prefill ----
// For callers that cannot allocate device memory (HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc): the records and the
// segment scratch live in one fixed device array instead of a caller
// workspace.  Every call on a GPU shares that GPU's array, so calls that
// overlap on one GPU (other streams, other threads) race; calls in order on
// one stream are safe.  Nothing in it has to start at zero: each call writes
// every record and segment state before reading it.
constexpr int64_t kNoAllocScratchBytes = GDN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxScratchDevices];

// The device address of `scratch` on the device the stream runs on.  The
// host-side name is only a stand-in; each device holds its own copy at its
// own address, looked up once per device with that device current.
int scratch_on(hipStream_t stream, uint8_t** out) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  int dev = cur;
  if (stream) {
    e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) return e;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) return GDN_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) {
      const hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return GDN_OK;
}

}  // namespace

// The bytes at the array's end hold the two token offsets of a sequence
// that runs in pieces (where the kernels read cu_seqlens).
constexpr int64_t kNoAllocCuBytes = 256;

namespace {
__global__ void set_cu_pair_kernel(int64_t* dst, int64_t t0, int64_t t1) {
  if (threadIdx.x == 0) {
    dst[0] = t0;
    dst[1] = t1;
  }
}
}  // namespace

// A call whose records do not fit the array runs as pieces in order on the
// stream, without segments: groups of whole sequences whose records fit (the
// kernels take the tokens' offsets from cu_seqlens, so a group only moves the
// cu_seqlens, slot-id and fresh pointers), and a sequence longer than the
// array holds as token ranges of whole chunks, each one starting from the
// state (hT) and conv taps the range before it left in the pools -- what two
// prefill calls over those ranges would do.  Planning needs the host offsets
// (cu_seqlens_host); a sequence in ranges needs its final state stored (hT).
extern "C" int gdn_conv_chunk_prefill_noalloc(const uint16_t* x, int64_t sx_row, uint16_t* conv_state,
                                              int64_t ss_seq, int64_t ss_ch, const uint16_t* conv_w,
                                              const uint16_t* b, const uint16_t* a, const void* A_log,
                                              const void* dt_bias, int param_is_fp32, const float* h0, float* hT,
                                              const int64_t* state_ids, const uint8_t* fresh, int64_t state_stride,
                                              const int64_t* cu_seqlens, const int64_t* cu_seqlens_host,
                                              int max_segments, int n_seqs, int64_t N, int Hk, int Hv, int D,
                                              float scale, int l2norm, uint16_t* o, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (n_seqs < 0 || N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return GDN_ERR_INVALID_ARG;
  if (n_seqs == 0) return GDN_OK;
  const int64_t need = gdn_conv_chunk_prefill_workspace_size(N, n_seqs, Hv, D);
  if (need < 0) return GDN_ERR_INVALID_ARG;
  constexpr int64_t kCap = kNoAllocScratchBytes - kNoAllocCuBytes;
  const int64_t rec = static_cast<int64_t>(Hv) * rec_bytes(D);  // one chunk's records
  const int64_t cap_chunks = kCap / rec;
  if (need > kCap && (!cu_seqlens_host || cap_chunks < 2)) return GDN_ERR_SCRATCH;
  int st = conv_chunk_check(x, sx_row, conv_state, ss_seq, ss_ch, conv_w, b, a, A_log, dt_bias, h0, hT,
                            state_stride, cu_seqlens, cu_seqlens_host, max_segments, kPhasePrep | kPhaseState,
                            nullptr, n_seqs, Hk, Hv, D, o);
  if (st != GDN_OK) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (need <= kCap) {
    // one call, as the workspace entry point runs it
    uint8_t* ws = nullptr;
    if ((st = scratch_on(s, &ws)) != GDN_OK) return st;
    const int64_t nc_bound = (N + kC - 1) / kC + n_seqs;
    uint8_t* seg_ws = seg_scratch_bytes(n_seqs, Hv, D) ? ws + nc_bound * rec : nullptr;
    return conv_chunk_run(x, sx_row, conv_state, ss_seq, ss_ch, conv_w, b, a, A_log, dt_bias, param_is_fp32, h0,
                          hT, state_ids, fresh, state_stride, cu_seqlens, cu_seqlens_host, max_segments,
                          kPhasePrep | kPhaseState, nullptr, n_seqs, N, Hk, Hv, D, scale, l2norm, o, ws, seg_ws, s);
  }
  // the plan, checked before anything launches
  for (int r = 0; r < n_seqs; ++r) {
    const int64_t len = cu_seqlens_host[r + 1] - cu_seqlens_host[r];
    if (len < 0) return GDN_ERR_INVALID_ARG;
    if (chunks_of(len) + 1 > cap_chunks && !hT) return GDN_ERR_SCRATCH;
  }
  uint8_t* ws = nullptr;
  if ((st = scratch_on(s, &ws)) != GDN_OK) return st;
  int64_t* cu_pair = reinterpret_cast<int64_t*>(ws + kCap);
  auto piece = [&](const float* p_h0, const int64_t* p_ids, const uint8_t* p_fresh, const int64_t* p_cu,
                   const int64_t* p_cu_host, int p_n, int64_t p_N) {
    return conv_chunk_run(x, sx_row, conv_state, ss_seq, ss_ch, conv_w, b, a, A_log, dt_bias, param_is_fp32, p_h0,
                          hT, p_ids, p_fresh, state_stride, p_cu, p_cu_host, 1, kPhasePrep | kPhaseState, nullptr,
                          p_n, p_N, Hk, Hv, D, scale, l2norm, o, ws, nullptr, s);
  };
  for (int r = 0; r < n_seqs;) {
    const int64_t* ids_r = state_ids ? state_ids + r : nullptr;
    const uint8_t* fresh_r = fresh ? fresh + r : nullptr;
    const int64_t t_beg = cu_seqlens_host[r], t_end = cu_seqlens_host[r + 1];
    if (chunks_of(t_end - t_beg) + 1 > cap_chunks) {
      // one sequence, token ranges of cap_chunks - 1 whole chunks
      const int64_t step = (cap_chunks - 1) * kC;
      for (int64_t t0 = t_beg; t0 < t_end; t0 += step) {
        const int64_t t1 = std::min(t0 + step, t_end);
        set_cu_pair_kernel<<<dim3(1), dim3(64), 0, s>>>(cu_pair, t0, t1);
        if ((st = gdn_launch_status()) != GDN_OK) return st;
        const int64_t cu_h[2] = {t0, t1};
        const bool first = t0 == t_beg;
        if ((st = piece(first ? h0 : hT, ids_r, first ? fresh_r : nullptr, cu_pair, cu_h, 1, t1 - t0)) != GDN_OK)
          return st;
      }
      ++r;
      continue;
    }
    // the longest run of whole sequences from r whose records fit
    int r1 = r + 1;
    while (r1 < n_seqs && chunks_of(cu_seqlens_host[r1 + 1] - t_beg) + (r1 + 1 - r) <= cap_chunks &&
           chunks_of(cu_seqlens_host[r1 + 1] - cu_seqlens_host[r1]) + 1 <= cap_chunks)
      ++r1;
    if ((st = piece(h0, ids_r, fresh_r, cu_seqlens + r, cu_seqlens_host + r, r1 - r,
                    cu_seqlens_host[r1] - t_beg)) != GDN_OK)
      return st;
    r = r1;
  }
  return GDN_OK;
}
