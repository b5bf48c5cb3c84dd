// Chunked gated delta rule over packed varlen sequences, chunk size 64,
// fully fused: one workgroup walks all chunks of one (sequence, value head,
// v-block) and keeps its slice of the fp32 recurrent state in registers.
//
// Per chunk (rows t, s in [0, 64); G = inclusive cumsum of g in the chunk,
// gamma = G[63]; k^, q^ = L2-normalised rows; follows the torch port at
// nanovllm/models/qwen3_5.py:152-227):
//   L    = strict_lower( beta_t k^_t.k^_s e^{G_t-G_s} )
//   T    = (I + L)^-1                       (the reference's forward substitution)
//   W    = T diag(beta e^G) K^,   U = T diag(beta) V
//   Vn   = U - W S
//   O    = diag(e^G) Q^ S + lower_incl( q^_t.k^_s e^{G_t-G_s} ) Vn
//   S   <- e^gamma S + K^T diag(e^{gamma-G}) Vn
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

template <int D, int NW>
struct __align__(16) ChunkSmem {
  uint16_t Kt[D][kC + 8];       // K^T of the chunk (raw bf16), row = key dim
  uint16_t Qs[kC][D + 8];       // Q of the chunk (raw bf16), row = token
  uint16_t KrW[kC][D + 8];      // K row-major (phases 1-2), then W (phases 5-6)
  uint16_t Tp[kC][kC + 8];      // T' = T diag(beta rk e^G), bf16
  uint16_t Uh[kC][kC + 8];      // T'' = T diag(beta), hi
  uint16_t Ul[kC][kC + 8];      //                     lo
  uint16_t Ah[kC][kC + 8];      // A_qk hi
  uint16_t Al[kC][kC + 8];      // A_qk lo
  float Lf[kC][kC + 4];         // L (fp32)
  float Tf[kC][kC + 4];         // T (fp32), lower blocks only
  float scr[4][16][20];         // per-wave 16x16 scratch of the solve
  float G[kC], bt[kC], rk[kC], rq[kC];
  float cW[kC], cQ[kC], cK[kC];
  float ssk[NW][kC];
  float ssq[kC];
  float eg_last;
};

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

// Global -> register prefetch of one chunk's operands (issued a chunk ahead).
template <int D, int NW>
struct Prefetch {
  static constexpr int NT = 64 * NW;
  static constexpr int SEG = D / 8;               // 16-byte segments per row
  static constexpr int KPRE = SEG / NW;           // K segments per lane (lane = token)
  static constexpr int QPRE = kC * SEG / NT;      // Q segments per thread (row-major)
  s16x8_t k[KPRE];
  s16x8_t q[QPRE];
  uint16_t v[16];  // one VGPR each: packing into vectors here would wait on the loads
  float g;
  uint16_t b;  // raw bf16 bits: converting here would force a wait on the load

  // Rows past the chunk end are loaded from the last valid row (always in
  // bounds, no branches) and zeroed only where the chunk is staged, so no
  // instruction consumes a loaded value before the next chunk begins.
  __device__ __forceinline__ void load(const uint16_t* qh, int64_t sq, const uint16_t* kh, int64_t sk,
                                       const uint16_t* vh, int64_t sv, const float* gp, const uint16_t* bp,
                                       int Hv, int h, int64_t tok0, int len, int tid, int wave, int lane,
                                       int lg, int vcol) {
    const int last = len - 1;
#pragma unroll
    for (int j = 0; j < KPRE; ++j) {
      const int c8 = wave + NW * j;
      k[j] = *reinterpret_cast<const s16x8_t*>(kh + (tok0 + min(lane, last)) * sk + c8 * 8);
    }
#pragma unroll
    for (int j = 0; j < QPRE; ++j) {
      const int e = tid + NT * j;
      const int t = e / SEG, c8 = e % SEG;
      q[j] = *reinterpret_cast<const s16x8_t*>(qh + (tok0 + min(t, last)) * sq + c8 * 8);
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int s = 32 * kt + 8 * lg + i;
        v[8 * kt + i] = vh[(tok0 + min(s, last)) * sv + vcol];
      }
    const int64_t gi = (tok0 + min(lane, last)) * Hv + h;
    g = gp[gi];
    b = bp[gi];
  }
};

template <int D, int NW>
__global__ __launch_bounds__(64 * NW) void chunk_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t sq, const uint16_t* __restrict__ k, int64_t sk,
    const uint16_t* __restrict__ v, int64_t sv, const float* __restrict__ g,
    const uint16_t* __restrict__ beta, const float* h0, float* hT, const int64_t* __restrict__ ids,
    int64_t sstride, const int64_t* __restrict__ cu, int n_seqs, int Hk, int Hv, float scale,
    int l2norm, uint16_t* __restrict__ o) {
  constexpr int NT = 64 * NW;
  constexpr int BV = 16 * NW;
  constexpr int NVB = D / BV;
  constexpr int KTD = D / 32;  // contraction steps over the key dim
  constexpr int MTD = D / 16;  // 16-row tiles over the key dim
  constexpr int LDF = kC + 4;
  using PF = Prefetch<D, NW>;
  static_assert(NW >= 4 && D % BV == 0, "chunk kernel shape");
  static_assert(PF::KPRE * NW == PF::SEG && PF::QPRE * NT == kC * PF::SEG, "prefetch tiling");

  __shared__ ChunkSmem<D, NW> sm;

  const int64_t wi = gdn::xcd_remap(blockIdx.x, static_cast<int64_t>(n_seqs) * Hv * NVB);
  if (wi < 0) return;
  const int vb = static_cast<int>(wi % NVB);
  const int h = static_cast<int>((wi / NVB) % Hv);
  const int r = static_cast<int>(wi / (static_cast<int64_t>(NVB) * Hv));
  const int kh = h / (Hv / Hk);

  const int64_t bos = cu[r];
  const int64_t seqlen = cu[r + 1] - bos;
  const uint16_t* qh = q + static_cast<int64_t>(kh) * D;
  const uint16_t* kh_ = k + static_cast<int64_t>(kh) * D;
  const uint16_t* vh = v + static_cast<int64_t>(h) * D;
  const int64_t srow = ids ? ids[r] : r;

  // state / output column of this lane: rows 16*mt + 4*(lane>>4) + i of S
  const int vcol0 = vb * BV + 16 * (threadIdx.x >> 6) + (threadIdx.x & 15);
  const int lg0 = (threadIdx.x & 63) >> 4;

  // ---- state slice: S[mt] holds rows 16mt + 4lg + i, column vcol ----
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

  PF pf;
  if (seqlen > 0)
    pf.load(qh, sq, kh_, sk, vh, sv, g, beta, Hv, h, bos, static_cast<int>(min<int64_t>(kC, seqlen)),
            threadIdx.x, threadIdx.x >> 6, threadIdx.x & 63, (threadIdx.x & 63) >> 4, vcol0);

  for (int64_t c0 = 0; c0 < seqlen; c0 += kC) {
    const int len = static_cast<int>(min<int64_t>(kC, seqlen - c0));
    const int64_t tok0 = bos + c0;
    // Re-derive the lane indices from an opaque copy each chunk.  Otherwise
    // the compiler hoists every lane-dependent LDS / global address of the
    // loop body out of the loop and keeps them all live in VGPRs, which
    // spills; rebuilt here they cost a few ALU ops per chunk instead.
    int tid_l = static_cast<int>(threadIdx.x);
    asm volatile("" : "+v"(tid_l));
    const int tid = tid_l;
    const int lane = tid_l & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid_l >> 6);
    const int vcol = vb * BV + 16 * wave + lr;
    __syncthreads();  // previous chunk's LDS readers are done

    // ---- phase 1: stage the prefetched chunk, row norms, gates ----
    s16x8_t vf[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        vf[kt][i] = 32 * kt + 8 * lg + i < len ? static_cast<short>(pf.v[8 * kt + i]) : static_cast<short>(0);
    {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < PF::KPRE; ++j) {
        const int c8 = wave + NW * j;
        const s16x8_t kv8 = lane < len ? pf.k[j] : zero8();
        *reinterpret_cast<s16x8_t*>(&sm.KrW[lane][c8 * 8]) = kv8;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint16_t bits = static_cast<uint16_t>(kv8[i]);
          sm.Kt[c8 * 8 + i][lane] = bits;
          const float f = gdn::bf2f(bits);
          ss += f * f;
        }
      }
      sm.ssk[wave][lane] = ss;
#pragma unroll
      for (int j = 0; j < PF::QPRE; ++j) {
        const int e = tid + NT * j;
        const int t = e / PF::SEG, c8 = e % PF::SEG;
        const s16x8_t qv8 = t < len ? pf.q[j] : zero8();
        *reinterpret_cast<s16x8_t*>(&sm.Qs[t][c8 * 8]) = qv8;
        float qs = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float f = gdn::bf2f(static_cast<uint16_t>(qv8[i]));
          qs += f * f;
        }
#pragma unroll
        for (int m = PF::SEG / 2; m >= 1; m >>= 1) qs += __shfl_xor(qs, m, 64);
        if (c8 == 0) sm.ssq[t] = qs;
      }
      if (wave == 0) {
        float gv = lane < len ? pf.g : 0.f;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
          const float o_ = __shfl_up(gv, d, 64);
          if (lane >= d) gv += o_;
        }
        sm.G[lane] = gv;
        sm.bt[lane] = lane < len ? gdn::bf2f(pf.b) : 0.f;
      }
    }
    // issue the next chunk's loads now: their latency hides behind this chunk
    if (c0 + kC < seqlen)
      pf.load(qh, sq, kh_, sk, vh, sv, g, beta, Hv, h, tok0 + kC,
              static_cast<int>(min<int64_t>(kC, seqlen - c0 - kC)), tid, wave, lane, lg, vcol);
    __syncthreads();
    if (tid < kC) {
      const int t = tid;
      float ssk = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) ssk += sm.ssk[w][t];
      const float rk = l2norm ? rsqrtf(ssk + 1e-6f) : 1.0f;
      const float rq = l2norm ? rsqrtf(sm.ssq[t] + 1e-6f) : 1.0f;
      const float Gt = sm.G[t];
      const float Gl = sm.G[kC - 1];
      sm.rk[t] = rk;
      sm.rq[t] = rq;
      sm.cW[t] = sm.bt[t] * rk * expf(Gt);
      sm.cQ[t] = rq * scale * expf(Gt);
      sm.cK[t] = rk * expf(Gl - Gt);
      if (t == 0) sm.eg_last = expf(Gl);
    }
    __syncthreads();

    // ---- phase 2a: K K^T -> L (fp32), lower-triangular tiles ----
    for (int j = wave; j < 10; j += NW) {
      int mt, nt;
      tri_tile(j, mt, nt);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < KTD; ++kt) {
        const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.KrW[16 * mt + lr][32 * kt + 8 * lg]);
        const s16x8_t b8 = *reinterpret_cast<const s16x8_t*>(&sm.KrW[16 * nt + lr][32 * kt + 8 * lg]);
        acc = gdn::mfma16x16x32(a8, b8, acc);
      }
      const int s = 16 * nt + lr;
      const float rks = sm.rk[s];
      const float Gs = sm.G[s];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * mt + 4 * lg + i;
        sm.Lf[t][s] = s < t ? acc[i] * sm.bt[t] * sm.rk[t] * rks * expf(sm.G[t] - Gs) : 0.f;
      }
    }
    __syncthreads();

    // ---- phase 2b / solve step 1: wave 0 inverts the diagonal blocks while
    //      the other waves form A_qk = lower(Q K^T) (hi/lo) ----
    if (wave == 0) {
      const int bb = lane >> 4, c = lane & 15, base = 16 * bb;
      float x[16];
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const float4* lrow = reinterpret_cast<const float4*>(&sm.Lf[base + rr][base]);
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
      for (int rr = 0; rr < 16; ++rr) sm.Tf[base + rr][base + c] = x[rr];
    } else {
      for (int j = wave - 1; j < 10; j += NW - 1) {
        int mt, nt;
        tri_tile(j, mt, nt);
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < KTD; ++kt) {
          const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.Qs[16 * mt + lr][32 * kt + 8 * lg]);
          const s16x8_t b8 = *reinterpret_cast<const s16x8_t*>(&sm.KrW[16 * nt + lr][32 * kt + 8 * lg]);
          acc = gdn::mfma16x16x32(a8, b8, acc);
        }
        const int s = 16 * nt + lr;
        const float rks = sm.rk[s] * scale;
        const float Gs = sm.G[s];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * mt + 4 * lg + i;
          const float a = s <= t ? acc[i] * sm.rq[t] * rks * expf(sm.G[t] - Gs) : 0.f;
          uint16_t hi, lo;
          gdn::split_bf16(a, hi, lo);
          sm.Ah[t][s] = hi;
          sm.Al[t][s] = lo;
        }
      }
    }
    __syncthreads();
    // first sub-diagonal: T(j+1, j) = -T(j+1,j+1) L(j+1,j) T(j,j)
    if (wave < 3) {
      const int j = wave, i = j + 1;
      f32x4_t p = {0.f, 0.f, 0.f, 0.f};
      p = mm16_f32(p, &sm.Lf[16 * i][16 * j], LDF, &sm.Tf[16 * j][16 * j], LDF, lane);
      st16_f32(&sm.scr[wave][0][0], 20, p, 1.f, lane);
      wave_sync();
      f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
      t2 = mm16_f32(t2, &sm.Tf[16 * i][16 * i], LDF, &sm.scr[wave][0][0], 20, lane);
      st16_f32(&sm.Tf[16 * i][16 * j], LDF, t2, -1.f, lane);
    } else if (wave == 3) {
      f32x4_t p = {0.f, 0.f, 0.f, 0.f};
      p = mm16_f32(p, &sm.Lf[48][0], LDF, &sm.Tf[0][0], LDF, lane);  // L30 T00
      st16_f32(&sm.scr[3][0][0], 20, p, 1.f, lane);
    }
    __syncthreads();
    // second sub-diagonal: T20, T31; partial sum for T30
    if (wave == 0) {
      f32x4_t p = {0.f, 0.f, 0.f, 0.f};
      p = mm16_f32(p, &sm.Lf[32][0], LDF, &sm.Tf[0][0], LDF, lane);    // L20 T00
      p = mm16_f32(p, &sm.Lf[32][16], LDF, &sm.Tf[16][0], LDF, lane);  // L21 T10
      st16_f32(&sm.scr[0][0][0], 20, p, 1.f, lane);
      wave_sync();
      f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
      t2 = mm16_f32(t2, &sm.Tf[32][32], LDF, &sm.scr[0][0][0], 20, lane);
      st16_f32(&sm.Tf[32][0], LDF, t2, -1.f, lane);
    } else if (wave == 1) {
      f32x4_t p = {0.f, 0.f, 0.f, 0.f};
      p = mm16_f32(p, &sm.Lf[48][16], LDF, &sm.Tf[16][16], LDF, lane);  // L31 T11
      p = mm16_f32(p, &sm.Lf[48][32], LDF, &sm.Tf[32][16], LDF, lane);  // L32 T21
      st16_f32(&sm.scr[1][0][0], 20, p, 1.f, lane);
      wave_sync();
      f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
      t2 = mm16_f32(t2, &sm.Tf[48][48], LDF, &sm.scr[1][0][0], 20, lane);
      st16_f32(&sm.Tf[48][16], LDF, t2, -1.f, lane);
    } else if (wave == 3) {
      f32x4_t p = ld16_f32(&sm.scr[3][0][0], 20, lane);
      p = mm16_f32(p, &sm.Lf[48][16], LDF, &sm.Tf[16][0], LDF, lane);  // + L31 T10
      st16_f32(&sm.scr[3][0][0], 20, p, 1.f, lane);
    }
    __syncthreads();
    // third sub-diagonal: T30
    if (wave == 3) {
      f32x4_t p = ld16_f32(&sm.scr[3][0][0], 20, lane);
      p = mm16_f32(p, &sm.Lf[48][32], LDF, &sm.Tf[32][0], LDF, lane);  // + L32 T20
      st16_f32(&sm.scr[3][0][0], 20, p, 1.f, lane);
      wave_sync();
      f32x4_t t2 = {0.f, 0.f, 0.f, 0.f};
      t2 = mm16_f32(t2, &sm.Tf[48][48], LDF, &sm.scr[3][0][0], 20, lane);
      st16_f32(&sm.Tf[48][0], LDF, t2, -1.f, lane);
    }
    __syncthreads();

    // ---- phase 4: T' (bf16) and T'' (hi/lo), 4 columns per thread; zero the
    //      upper tiles of A_qk ----
    for (int e4 = tid; e4 < kC * (kC / 4); e4 += NT) {
      const int t = e4 >> 4, s0 = (e4 & 15) * 4;
      const bool lower = (s0 >> 4) <= (t >> 4);
      float4 tv = lower ? *reinterpret_cast<const float4*>(&sm.Tf[t][s0]) : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 cw = *reinterpret_cast<const float4*>(&sm.cW[s0]);
      const float4 cb = *reinterpret_cast<const float4*>(&sm.bt[s0]);
      uint2 tp;
      tp.x = gdn::f2bf2(tv.x * cw.x, tv.y * cw.y);
      tp.y = gdn::f2bf2(tv.z * cw.z, tv.w * cw.w);
      *reinterpret_cast<uint2*>(&sm.Tp[t][s0]) = tp;
      const float u0 = tv.x * cb.x, u1 = tv.y * cb.y, u2 = tv.z * cb.z, u3 = tv.w * cb.w;
      uint2 uh, ul;
      uh.x = gdn::f2bf2(u0, u1);
      uh.y = gdn::f2bf2(u2, u3);
      ul.x = gdn::f2bf2(u0 - lo_half(uh.x), u1 - hi_half(uh.x));
      ul.y = gdn::f2bf2(u2 - lo_half(uh.y), u3 - hi_half(uh.y));
      *reinterpret_cast<uint2*>(&sm.Uh[t][s0]) = uh;
      *reinterpret_cast<uint2*>(&sm.Ul[t][s0]) = ul;
      if (!lower) {
        *reinterpret_cast<uint2*>(&sm.Ah[t][s0]) = make_uint2(0u, 0u);
        *reinterpret_cast<uint2*>(&sm.Al[t][s0]) = make_uint2(0u, 0u);
      }
    }
    __syncthreads();

    // ---- phase 5: W = T' K (shared by all waves; overwrites K row-major) ----
    {
      constexpr int NJ = (4 * MTD + NW - 1) / NW;
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        const int j = wave + NW * jj;
        if (j >= 4 * MTD) break;
        const int mt = j % 4, nt = j / 4;
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const s16x8_t a8 = *reinterpret_cast<const s16x8_t*>(&sm.Tp[16 * mt + lr][32 * kt + 8 * lg]);
          const s16x8_t b8 = *reinterpret_cast<const s16x8_t*>(&sm.Kt[16 * nt + lr][32 * kt + 8 * lg]);
          acc = gdn::mfma16x16x32(a8, b8, acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) sm.KrW[16 * mt + 4 * lg + i][16 * nt + lr] = gdn::f2bf(acc[i]);
      }
    }
    __syncthreads();
    // ---- phase 6: per-wave state chain (registers only) ----
    {
      // W S and Q S with S split hi/lo per contraction step (key dim)
      f32x4_t ws[4], qs[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        ws[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        qs[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int kt = 0; kt < KTD; ++kt) {
        s16x8_t sh, sl;
        split_frag(S[2 * kt], S[2 * kt + 1], sh, sl);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const s16x8_t wa = perm_frag(&sm.KrW[16 * mt + lr][32 * kt], lg);
          const s16x8_t qa = perm_frag(&sm.Qs[16 * mt + lr][32 * kt], lg);
          ws[mt] = gdn::mfma16x16x32(wa, sh, ws[mt]);
          ws[mt] = gdn::mfma16x16x32(wa, sl, ws[mt]);
          qs[mt] = gdn::mfma16x16x32(qa, sh, qs[mt]);
          qs[mt] = gdn::mfma16x16x32(qa, sl, qs[mt]);
        }
      }
      // U = T'' V, Vn = U - W S, O_inter = diag(cQ) Q S
      f32x4_t vn[4], oo[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        f32x4_t u = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const s16x8_t ah = *reinterpret_cast<const s16x8_t*>(&sm.Uh[16 * mt + lr][32 * kt + 8 * lg]);
          const s16x8_t al = *reinterpret_cast<const s16x8_t*>(&sm.Ul[16 * mt + lr][32 * kt + 8 * lg]);
          u = gdn::mfma16x16x32(ah, vf[kt], u);
          u = gdn::mfma16x16x32(al, vf[kt], u);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * mt + 4 * lg + i;
          vn[mt][i] = u[i] - ws[mt][i];
          oo[mt][i] = sm.cQ[t] * qs[mt][i];
        }
      }
      // Vn and Vn' = diag(cK) Vn as B fragments (contraction over tokens)
      s16x8_t vh_[2], vl_[2], ph[2], pl[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        split_frag(vn[2 * kt], vn[2 * kt + 1], vh_[kt], vl_[kt]);
        f32x4_t p0, p1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p0[i] = vn[2 * kt][i] * sm.cK[32 * kt + 4 * lg + i];
          p1[i] = vn[2 * kt + 1][i] * sm.cK[32 * kt + 16 + 4 * lg + i];
        }
        split_frag(p0, p1, ph[kt], pl[kt]);
      }
      // O += A_qk Vn (lower-triangular: skip the all-zero upper k-steps)
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int ta = 16 * mt + lr;
        f32x4_t acc = oo[mt];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          if (32 * kt > 16 * mt + 15) break;
          const s16x8_t ah = perm_frag(&sm.Ah[ta][32 * kt], lg);
          const s16x8_t al = perm_frag(&sm.Al[ta][32 * kt], lg);
          acc = gdn::mfma16x16x32(ah, vh_[kt], acc);
          acc = gdn::mfma16x16x32(ah, vl_[kt], acc);
          acc = gdn::mfma16x16x32(al, vh_[kt], acc);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * mt + 4 * lg + i;
          if (t < len) o[((tok0 + t) * Hv + h) * D + vcol] = gdn::f2bf(acc[i]);
        }
      }
      // S <- e^gamma S + K^T Vn'
      const float eg = sm.eg_last;
#pragma unroll
      for (int mt = 0; mt < MTD; ++mt) {
        f32x4_t acc;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = S[mt][i] * eg;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
          const s16x8_t ka = perm_frag(&sm.Kt[16 * mt + lr][32 * kt], lg);
          acc = gdn::mfma16x16x32(ka, ph[kt], acc);
          acc = gdn::mfma16x16x32(ka, pl[kt], acc);
        }
        S[mt] = acc;
      }
    }
  }

  if (hT) {
    float* hp = hT + srow * sstride + static_cast<int64_t>(h) * D * D + vcol0;
#pragma unroll
    for (int mt = 0; mt < MTD; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) hp[static_cast<int64_t>(16 * mt + 4 * lg0 + i) * D] = S[mt][i];
  }
}

template <int D, int NW>
int launch_chunk(const uint16_t* q, int64_t sq, const uint16_t* k, int64_t sk, const uint16_t* v,
                 int64_t sv, const float* g, const uint16_t* beta, const float* h0, float* hT,
                 const int64_t* ids, int64_t sstride, const int64_t* cu, int n_seqs, int Hk,
                 int Hv, float scale, int l2norm, uint16_t* o, hipStream_t stream) {
  constexpr int NVB = D / (16 * NW);
  const int64_t work = static_cast<int64_t>(n_seqs) * Hv * NVB;
  const int64_t grid = gdn::kNumXcd * ((work + gdn::kNumXcd - 1) / gdn::kNumXcd);
  chunk_prefill_kernel<D, NW><<<dim3(static_cast<unsigned>(grid)), dim3(64 * NW), 0, stream>>>(
      q, sq, k, sk, v, sv, g, beta, h0, hT, ids, sstride, cu, n_seqs, Hk, Hv, scale, l2norm, o);
  return gdn_launch_status();
}

}  // namespace

extern "C" int gdn_chunk_prefill(const uint16_t* q, int64_t sq_tok, const uint16_t* k,
                                 int64_t sk_tok, const uint16_t* v, int64_t sv_tok, const float* g,
                                 const uint16_t* beta, const float* h0, float* hT,
                                 const int64_t* state_ids, int64_t state_stride,
                                 const int64_t* cu_seqlens, int n_seqs, int64_t N, int Hk, int Hv,
                                 int D, float scale, int l2norm, uint16_t* o, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (n_seqs < 0 || N < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return GDN_ERR_INVALID_ARG;
  if (n_seqs == 0) return GDN_OK;
  if (!q || !k || !v || !g || !beta || !cu_seqlens || !o) return GDN_ERR_INVALID_ARG;
  // 16-byte row fragments of q / k and float state rows
  if (sq_tok % 8 || sk_tok % 8 || reinterpret_cast<uintptr_t>(q) % 16 ||
      reinterpret_cast<uintptr_t>(k) % 16 || ((h0 || hT) && state_stride < static_cast<int64_t>(Hv) * D * D))
    return GDN_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128)
    return launch_chunk<128, 8>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids,
                                state_stride, cu_seqlens, n_seqs, Hk, Hv, scale, l2norm, o, s);
  return launch_chunk<64, 4>(q, sq_tok, k, sk_tok, v, sv_tok, g, beta, h0, hT, state_ids,
                             state_stride, cu_seqlens, n_seqs, Hk, Hv, scale, l2norm, o, s);
}
