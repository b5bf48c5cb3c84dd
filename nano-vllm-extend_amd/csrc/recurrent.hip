// Recurrent gated delta rule for decode (T >= 1 tokens per sequence) against
// a slot-indexed fp32 state pool, plus the speculative-verify state commit.
//
// Math per token (nanovllm/models/qwen3_5.py:575-594, :616-651):
//   q, k L2-normalised in fp32 (eps 1e-6), q *= scale
//   S <- S * exp(g);  kv = S^T k;  delta = beta * (v - kv);  S <- S + k delta^T
//   o = S^T q  =  (S*exp(g))^T q + delta * (k . q)
// The last identity lets one cross-wave reduction pass produce both kv and o.
//
// HBM-bound: the D x D fp32 state tile of each (sequence, head) is read once
// into registers and written once (plus optional per-token states).  The
// state stores are non-temporal, and so are the state loads of one-token
// decode: a layer's states come back only after every other layer's have
// streamed through, so allocating them in the caches only evicts other data
// (an in-place pass over config 2's tiles: 108 us with cached loads, 96 us
// with non-temporal ones).  The multi-token form keeps cached loads (its
// start states were often written by the previous step: 104 us cached, 130 us
// non-temporal at config 4).  One workgroup of 64 * NW threads owns a
// (sequence, head, v-block) tile of D x VB columns, VB = D / NVB; each thread
// holds float4 column groups of NP rows so every wave access is a contiguous
// run of VB*4 bytes per row.  One-token decode of whole-head tiles (NVB = 1,
// D = 128) runs 8 waves (config 2: 103.4 us at 4 waves, 101.4 us at 8; 16
// waves need more registers than two workgroups per CU leave and measured
// 118.7 us).
#include "gdn_common.h"

namespace {

// State tiles move through raw buffer loads and stores: the tile base in the
// descriptor (uniform over the workgroup), the lane's offset in one VGPR and
// the pass's offset as an immediate, so the NP row passes need no address
// registers of their own.  The range is left open (offsets stay inside the
// D x D tile); stores are non-temporal (cache policy bit nt).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const float* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), static_cast<short>(0), 0x7fffffff, 0x00020000);
}
template <int kPolicy>
__device__ __forceinline__ float4 tile_ld(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kPolicy));
}
constexpr int kLoadCached = 0;
constexpr int kLoadNT = 2;  // non-temporal (cache policy bit nt)
__device__ __forceinline__ void tile_st_nt(__amdgpu_buffer_rsrc_t r, int voff, int soff, const float4& v) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, voff, soff, 2);
}

// Inputs of the fused decode step (one token per sequence): the gates from
// their raw inputs, and the v channels' conv with its state roll from the raw
// rows, computed in the kernel (q and k come from the decode conv as usual).
// Each v channel belongs to one workgroup, so its roll races with no reader.
struct DecodeIn {
  const uint16_t* xv;      // raw rows at the first v channel, row stride sx (NULL: not fused)
  int64_t sx;
  uint16_t* vpool;         // conv state pool at the first v channel: slot s, channel c, tap j
  int64_t sp_slot, sp_ch;  //   at vpool + s*sp_slot + c*sp_ch + j
  const uint16_t* wv;      // [Hv*D, 4] conv taps of the v channels
  const uint16_t* a;       // [B, Hv] gate inputs
  const uint16_t* b;
  const void* A_log;       // [Hv], bf16 or fp32 (param_f32)
  const void* dt_bias;
  int param_f32;
  // q and k from their raw channels too (NULL: from the q / k arguments):
  // the decode conv of head kh's q and k channels and their roll, by wave 0.
  // Only with Hk == Hv and whole heads per workgroup, so each of these
  // channels belongs to one workgroup as well.
  const uint16_t* xqk;     // raw rows at channel 0, row stride sx
  uint16_t* qkpool;        // conv state pool at channel 0 (sp_slot, sp_ch)
  const uint16_t* wqk;     // [C, 4] conv taps from channel 0
  int key_dim;             // Hk * D: the first k channel
};

// Gated RMSNorm on the output (fused decode step, whole heads per workgroup):
// o receives bf16(norm_gate(bf16(core), r, w, z)) instead of the core output,
// the same bits as gdn_rmsnorm_gated on it.
struct NormIn {
  const uint16_t* z;  // [B, Hv*D] gate rows, row stride sz (NULL: no norm)
  int64_t sz;
  const uint16_t* w;  // [D]
  float eps;
};

// Initial states of a speculative-verify step taken from the previous step's
// per-token states (deferred commit): row b starts from src[b, acc[b] - 1]
// (src [B, T_src, Hv, D, D]) when 1 <= acc[b] <= T_src, else from its pool row.
struct SrcIn {
  const float* src;
  const int64_t* acc;  // NULL: every row from the pool
  int T_src;
};

template <int D, int NVB, int NW, bool kFused, int kPolicy>
__global__ __launch_bounds__(64 * NW) void recurrent_kernel(
    const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, const uint16_t* __restrict__ k,
    int64_t sk_b, int64_t sk_t, const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t,
    const float* __restrict__ g, const uint16_t* __restrict__ beta, const float* s_in,
    int64_t s_in_stride, float* s_out, int64_t s_out_stride, const int64_t* __restrict__ ids,
    float* __restrict__ inter, uint16_t* __restrict__ o, int B, int T, int Hk, int Hv,
    float scale, int l2norm, DecodeIn din, NormIn nin, SrcIn src) {
  constexpr int VB = D / NVB;       // state columns per workgroup
  constexpr int CPR = VB / 4;       // float4 column groups per row
  constexpr int RPP = 64 * NW / CPR;  // rows per pass of the workgroup
  constexpr int NP = D / RPP;     // passes (float4 registers per thread)
  static_assert(CPR <= 64 && 64 % CPR == 0 && NP >= 1, "tile shape");
  // the fused v conv gives each of the tile's VB columns a thread
  static_assert(!kFused || 64 * NW >= VB, "fused v conv: a thread per column");

  __shared__ float sq[2][D];
  __shared__ float sk[2][D];
  __shared__ float skq[2];
  __shared__ float red[2][NW][2][VB];
  __shared__ float tot[NW > 4 ? 2 : 1][2][VB];  // NW > 4: column totals of S^T k and S^T q
  __shared__ float svv[2][VB];                  // fused: the v channels' conv outputs

  const int64_t wi = gdn::xcd_remap(blockIdx.x, static_cast<int64_t>(B) * Hv * NVB);
  if (wi < 0) return;
  const int vb = static_cast<int>(wi % NVB);
  const int h = static_cast<int>((wi / NVB) % Hv);
  const int b = static_cast<int>(wi / (static_cast<int64_t>(NVB) * Hv));
  const int kh = h / (Hv / Hk);
  const int tid = threadIdx.x;
  const int c4 = tid % CPR;
  const int r0 = tid / CPR;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int col = vb * VB + c4 * 4;

  const int64_t row = ids ? ids[b] : b;
  // an accepted count outside [1, T_src] keeps the pool row, as the commit
  // kernel leaves such a row untouched
  const int64_t acc = src.acc ? src.acc[b] : 0;
  const bool from_src = acc >= 1 && acc <= src.T_src;
  const float* sin = from_src ? src.src + ((static_cast<int64_t>(b) * src.T_src + acc - 1) * Hv + h) * D * D
                              : s_in + row * s_in_stride + static_cast<int64_t>(h) * D * D;
  // byte offset of this lane's float4 in the tile, and of row pass j
  const int voff = (r0 * D + col) * 4;
  constexpr int kPass = RPP * D * 4;
  // Fused: the decode conv (one token) of the head's channels, one channel
  // per thread: with din.xqk thread t < 3 D takes channel t % D of part
  // t / D (q, k, v), else thread t < VB the v channel of column t.  Its raw
  // input, taps and weights are loaded ahead of the state tile so their
  // latency overlaps the tile's loads.
  int cpart = -1, cci = 0;
  if (kFused) {
    if (din.xqk) {
      if (tid < 3 * D) { cpart = tid / D; cci = tid % D; }
    } else if (tid < VB) {
      cpart = 2;
      cci = tid;
    }
  }
  const bool cv_v = cpart == 2;
  const int64_t cch = cv_v ? static_cast<int64_t>(h) * D + vb * VB + cci
                           : (cpart == 1 ? din.key_dim : 0) + static_cast<int64_t>(kh) * D + cci;
  uint16_t* ctap = nullptr;
  uint16_t cx = 0, cs[3] = {0, 0, 0};
  uint2 cw = make_uint2(0u, 0u);
  if (cpart >= 0) {
    cx = (cv_v ? din.xv : din.xqk)[static_cast<int64_t>(b) * din.sx + cch];
    ctap = (cv_v ? din.vpool : din.qkpool) + row * din.sp_slot + cch * din.sp_ch;
#pragma unroll
    for (int j = 0; j < 3; ++j) cs[j] = ctap[j];
    cw = *reinterpret_cast<const uint2*>((cv_v ? din.wv : din.wqk) + cch * 4);
  }
  // Fused (one token): the gate inputs, and the gate row and weight of the
  // norm epilogue, also go out ahead of the tile.
  uint16_t g_a = 0, g_b = 0;
  float g_alog = 0.f, g_dtb = 0.f;
  uint2 n_z = make_uint2(0u, 0u), n_w = make_uint2(0u, 0u);
  if constexpr (kFused) {
    const int64_t gi0 = static_cast<int64_t>(b) * Hv + h;
    g_a = din.a[gi0];
    g_b = din.b[gi0];
    g_alog = gdn::load_param(din.A_log, h, din.param_f32);
    g_dtb = gdn::load_param(din.dt_bias, h, din.param_f32);
    if (NVB == 1 && nin.z && r0 == 0) {
      n_z = *reinterpret_cast<const uint2*>(nin.z + static_cast<int64_t>(b) * nin.sz + static_cast<int64_t>(h) * D +
                                             col);
      n_w = *reinterpret_cast<const uint2*>(nin.w + col);
    }
  }
  // one load sequence (a branch between two would make the compiler wait for
  // the whole tile before the conv above can use its inputs)
  float4 S[NP];
  {
    const __amdgpu_buffer_rsrc_t r = tile_rsrc(sin);
#pragma unroll
    for (int j = 0; j < NP; ++j) S[j] = tile_ld<kPolicy>(r, voff, j * kPass);
  }

  for (int t = 0; t < T; ++t) {
    const int buf = t & 1;
    if (kFused) {
      // the conv of this thread's channel (the conv kernel's arithmetic, its
      // output rounded to bf16) into sq / sk / svv, then its roll (bit
      // copies; this thread alone reads and writes these taps).  One token.
      if (cpart >= 0) {
        const uint16_t* wsv = reinterpret_cast<const uint16_t*>(&cw);
        const float wk[4] = {gdn::bf2f(wsv[0]), gdn::bf2f(wsv[1]), gdn::bf2f(wsv[2]), gdn::bf2f(wsv[3])};
        const float y = gdn::bf2f(gdn::f2bf(
            gdn::conv_decode_silu(gdn::bf2f(cx), gdn::bf2f(cs[0]), gdn::bf2f(cs[1]), gdn::bf2f(cs[2]), wk)));
        float* dst = cpart == 0 ? &sq[buf][0] : cpart == 1 ? &sk[buf][0] : &svv[buf][0];
        dst[cci] = y;
        ctap[0] = cs[1];
        ctap[1] = cs[2];
        ctap[2] = cx;
      }
      if (din.xqk) __syncthreads();
    }
    // --- q, k of this token: wave 0 normalises and publishes them ---
    if (wave == 0) {
      constexpr int E = D / 64;
      const uint16_t* qp = q + static_cast<int64_t>(b) * sq_b + static_cast<int64_t>(t) * sq_t + static_cast<int64_t>(kh) * D;
      const uint16_t* kp = k + static_cast<int64_t>(b) * sk_b + static_cast<int64_t>(t) * sk_t + static_cast<int64_t>(kh) * D;
      float qf[E], kf[E];
      float qq = 0.f, kk = 0.f;
      if (kFused && din.xqk) {
        // the conv outputs from sq / sk (this lane's elements, overwritten
        // below with the normalised values)
#pragma unroll
        for (int e = 0; e < E; ++e) {
          qf[e] = sq[buf][lane * E + e];
          kf[e] = sk[buf][lane * E + e];
          qq += qf[e] * qf[e];
          kk += kf[e] * kf[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          qf[e] = gdn::bf2f(qp[lane * E + e]);
          kf[e] = gdn::bf2f(kp[lane * E + e]);
          qq += qf[e] * qf[e];
          kk += kf[e] * kf[e];
        }
      }
      qq = gdn::wave_sum(qq);
      kk = gdn::wave_sum(kk);
      const float rq = l2norm ? rsqrtf(qq + 1e-6f) : 1.0f;
      const float rk = l2norm ? rsqrtf(kk + 1e-6f) : 1.0f;
      float kq = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float qn = (qf[e] * rq) * scale;
        const float kn = kf[e] * rk;
        sq[buf][lane * E + e] = qn;
        sk[buf][lane * E + e] = kn;
        kq += qn * kn;
      }
      kq = gdn::wave_sum(kq);
      if (lane == 0) skq[buf] = kq;
    }
    const int64_t gi = (static_cast<int64_t>(b) * T + t) * Hv + h;
    float eg, bt;
    float vv[4];
    if constexpr (kFused) {
      // the gate kernel's arithmetic (g in fp32, beta rounded to bf16); one token
      eg = expf(gdn::gate_g(gdn::bf2f(g_a), g_alog, g_dtb));
      bt = gdn::bf2f(gdn::gate_beta(gdn::bf2f(g_b)));
    } else {
      eg = expf(g[gi]);
      bt = gdn::bf2f(beta[gi]);
      const uint16_t* vp = v + static_cast<int64_t>(b) * sv_b + static_cast<int64_t>(t) * sv_t + static_cast<int64_t>(h) * D + col;
      const uint2 u = *reinterpret_cast<const uint2*>(vp);
      const uint16_t* us = reinterpret_cast<const uint16_t*>(&u);
#pragma unroll
      for (int i = 0; i < 4; ++i) vv[i] = gdn::bf2f(us[i]);
    }
    __syncthreads();
    if constexpr (kFused) {
#pragma unroll
      for (int i = 0; i < 4; ++i) vv[i] = svv[buf][c4 * 4 + i];
    }

    // --- decay, then partial S^T k and S^T q over this thread's rows ---
    float kv[4] = {0.f, 0.f, 0.f, 0.f}, qv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const float kr = sk[buf][r0 + RPP * j];
      const float qr = sq[buf][r0 + RPP * j];
      S[j].x *= eg; S[j].y *= eg; S[j].z *= eg; S[j].w *= eg;
      kv[0] += S[j].x * kr; kv[1] += S[j].y * kr; kv[2] += S[j].z * kr; kv[3] += S[j].w * kr;
      qv[0] += S[j].x * qr; qv[1] += S[j].y * qr; qv[2] += S[j].z * qr; qv[3] += S[j].w * qr;
    }
#pragma unroll
    for (int m = CPR; m < 64; m <<= 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kv[i] += __shfl_xor(kv[i], m, 64);
        qv[i] += __shfl_xor(qv[i], m, 64);
      }
    }
    if (lane < CPR) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        red[buf][wave][0][c4 * 4 + i] = kv[i];
        red[buf][wave][1][c4 * 4 + i] = qv[i];
      }
    }
    __syncthreads();

    // --- delta, state update, output ---
    const float kq = skq[buf];
    float delta[4], out[4];
    if constexpr (NW > 4) {
      // the wave partials summed once per column (waves in order), then read
      // back by every thread
      if (tid < 2 * VB) {
        const int sel = tid / VB, c = tid % VB;
        float acc = red[buf][0][sel][c];
#pragma unroll
        for (int w = 1; w < NW; ++w) acc += red[buf][w][sel][c];
        tot[0][sel][c] = acc;
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        delta[i] = (vv[i] - tot[0][0][c4 * 4 + i]) * bt;
        out[i] = tot[0][1][c4 * 4 + i] + delta[i] * kq;
      }
      // (tot is rewritten only after the next token's first barrier)
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float kvt = red[buf][0][0][c4 * 4 + i], qvt = red[buf][0][1][c4 * 4 + i];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
          kvt += red[buf][w][0][c4 * 4 + i];
          qvt += red[buf][w][1][c4 * 4 + i];
        }
        delta[i] = (vv[i] - kvt) * bt;
        out[i] = qvt + delta[i] * kq;
      }
    }
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const float kr = sk[buf][r0 + RPP * j];
      S[j].x += kr * delta[0]; S[j].y += kr * delta[1]; S[j].z += kr * delta[2]; S[j].w += kr * delta[3];
    }
    if (inter) {
      const __amdgpu_buffer_rsrc_t r =
          tile_rsrc(inter + ((static_cast<int64_t>(b) * T + t) * Hv + h) * static_cast<int64_t>(D) * D);
#pragma unroll
      for (int j = 0; j < NP; ++j) tile_st_nt(r, voff, j * kPass, S[j]);
    }
    if (s_out && t == T - 1) {
      // the final state goes out before the output epilogue
      const __amdgpu_buffer_rsrc_t r = tile_rsrc(s_out + row * s_out_stride + static_cast<int64_t>(h) * D * D);
#pragma unroll
      for (int j = 0; j < NP; ++j) tile_st_nt(r, voff, j * kPass, S[j]);
    }
    if (r0 == 0) {
      uint2 u;
      uint16_t* us = reinterpret_cast<uint16_t*>(&u);
#pragma unroll
      for (int i = 0; i < 4; ++i) us[i] = gdn::f2bf(out[i]);
      if (NVB == 1 && nin.z) {
        // the row's D outputs sit in lanes 0 .. D/4 - 1 of wave 0, 4 each.
        // mean(x^2) is summed in the standalone norm's order: 8 consecutive
        // values per group (this lane's and its pair's, lower columns
        // first), then a butterfly over the D/8 groups.
        float x[4], pr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = gdn::bf2f(us[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) pr[i] = __shfl_xor(x[i], 1, 64);
        const bool lo = (c4 & 1) == 0;
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) ss += (lo ? x[i] : pr[i]) * (lo ? x[i] : pr[i]);
#pragma unroll
        for (int i = 0; i < 4; ++i) ss += (lo ? pr[i] : x[i]) * (lo ? pr[i] : x[i]);
#pragma unroll
        for (int m = D / 16; m >= 1; m >>= 1) ss += __shfl_xor(ss, 2 * m, 64);
        const float r = rsqrtf(ss / static_cast<float>(D) + nin.eps);
        const uint16_t* zs = reinterpret_cast<const uint16_t*>(&n_z);
        const uint16_t* ws = reinterpret_cast<const uint16_t*>(&n_w);
        u.x = gdn::f2bf2(gdn::norm_gate(x[0], r, gdn::bf2f(ws[0]), gdn::bf2f(zs[0])),
                         gdn::norm_gate(x[1], r, gdn::bf2f(ws[1]), gdn::bf2f(zs[1])));
        u.y = gdn::f2bf2(gdn::norm_gate(x[2], r, gdn::bf2f(ws[2]), gdn::bf2f(zs[2])),
                         gdn::norm_gate(x[3], r, gdn::bf2f(ws[3]), gdn::bf2f(zs[3])));
      }
      *reinterpret_cast<uint2*>(o + gi * D + col) = u;
    }
  }
}

// pool[ids[b]] <- inter[b, accepted[b]-1]  (accepted 0: untouched).
// grid = B * Hv blocks of 256 threads, float4 copies.
__global__ __launch_bounds__(256) void state_commit_kernel(float* __restrict__ pool, int64_t slot_stride,
                                                           const int64_t* __restrict__ ids,
                                                           const float* __restrict__ inter,
                                                           const int32_t* __restrict__ accepted,
                                                           int T, int Hv, int D) {
  const int b = blockIdx.x / Hv;
  const int h = blockIdx.x % Hv;
  const int a = accepted[b];
  if (a <= 0 || a > T) return;
  const float4* src = reinterpret_cast<const float4*>(
      inter + ((static_cast<int64_t>(b) * T + (a - 1)) * Hv + h) * D * D);
  float4* dst = reinterpret_cast<float4*>(pool + ids[b] * slot_stride + static_cast<int64_t>(h) * D * D);
  for (int i = threadIdx.x; i < D * D / 4; i += 256) dst[i] = src[i];
}

// Measurement pass: each selected state tile read into registers and written
// back unchanged, with the one-token decode kernel's layout (NVB = 1; 8 waves
// at D = 128), cache policy and barrier between the loads and the stores: one
// decode step's state traffic without its arithmetic.  With dst != src the tiles land at
// the same offsets of a second pool (the out-of-place form of the same pass).
template <int D, int NT>
__global__ __launch_bounds__(NT) void state_tile_pass_kernel(const float* src, float* dst, int64_t slot_stride,
                                                             const int64_t* __restrict__ ids, int B, int Hv) {
  constexpr int CPR = D / 4;
  constexpr int RPP = NT / CPR;
  constexpr int NP = D / RPP;
  constexpr int kPass = RPP * D * 4;
  const int64_t wi = gdn::xcd_remap(blockIdx.x, static_cast<int64_t>(B) * Hv);
  if (wi < 0) return;
  const int h = static_cast<int>(wi % Hv);
  const int b = static_cast<int>(wi / Hv);
  const int64_t off = ids[b] * slot_stride + static_cast<int64_t>(h) * D * D;
  const __amdgpu_buffer_rsrc_t r = tile_rsrc(src + off);
  const __amdgpu_buffer_rsrc_t w = tile_rsrc(dst + off);
  const int voff = ((threadIdx.x / CPR) * D + (threadIdx.x % CPR) * 4) * 4;
  float4 S[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) S[j] = tile_ld<kLoadNT>(r, voff, j * kPass);
  __syncthreads();
#pragma unroll
  for (int j = 0; j < NP; ++j) tile_st_nt(w, voff, j * kPass, S[j]);
}

template <int D, int NVB, int NW, int kPolicy>
int launch_recurrent_t(const uint16_t* q, int64_t sq_b, int64_t sq_t, const uint16_t* k, int64_t sk_b,
                     int64_t sk_t, const uint16_t* v, int64_t sv_b, int64_t sv_t, const float* g,
                     const uint16_t* beta, const float* s_in, int64_t s_in_stride, float* s_out,
                     int64_t s_out_stride, const int64_t* ids, float* inter, uint16_t* o, int B,
                     int T, int Hk, int Hv, float scale, int l2norm, const DecodeIn& din, const NormIn& nin,
                     const SrcIn& src, hipStream_t stream) {
  // the fused conv gives each of a head's channels a thread
  if (din.xqk && (NVB != 1 || 64 * NW < 3 * D)) return GDN_ERR_INVALID_ARG;
  const int64_t work = static_cast<int64_t>(B) * Hv * NVB;
  const int64_t grid = gdn::kNumXcd * ((work + gdn::kNumXcd - 1) / gdn::kNumXcd);
  if (din.xv)
    recurrent_kernel<D, NVB, NW, true, kPolicy><<<dim3(static_cast<unsigned>(grid)), dim3(64 * NW), 0, stream>>>(
        q, sq_b, sq_t, k, sk_b, sk_t, v, sv_b, sv_t, g, beta, s_in, s_in_stride, s_out, s_out_stride,
        ids, inter, o, B, T, Hk, Hv, scale, l2norm, din, nin, src);
  else
    recurrent_kernel<D, NVB, NW, false, kPolicy><<<dim3(static_cast<unsigned>(grid)), dim3(64 * NW), 0, stream>>>(
        q, sq_b, sq_t, k, sk_b, sk_t, v, sv_b, sv_t, g, beta, s_in, s_in_stride, s_out, s_out_stride,
        ids, inter, o, B, T, Hk, Hv, scale, l2norm, din, nin, src);
  return gdn_launch_status();
}


// One token: non-temporal state loads on NW1 waves; more tokens: cached
// loads on 4 waves.
template <int D, int NVB, int NW1 = 4>
int launch_recurrent(const uint16_t* q, int64_t sq_b, int64_t sq_t, const uint16_t* k, int64_t sk_b,
                     int64_t sk_t, const uint16_t* v, int64_t sv_b, int64_t sv_t, const float* g,
                     const uint16_t* beta, const float* s_in, int64_t s_in_stride, float* s_out,
                     int64_t s_out_stride, const int64_t* ids, float* inter, uint16_t* o, int B,
                     int T, int Hk, int Hv, float scale, int l2norm, const DecodeIn& din, const NormIn& nin,
                     const SrcIn& src, hipStream_t stream) {
  if (T == 1)
    return launch_recurrent_t<D, NVB, NW1, kLoadNT>(q, sq_b, sq_t, k, sk_b, sk_t, v, sv_b, sv_t, g, beta, s_in,
                                                    s_in_stride, s_out, s_out_stride, ids, inter, o, B, T, Hk, Hv,
                                                    scale, l2norm, din, nin, src, stream);
  return launch_recurrent_t<D, NVB, 4, kLoadCached>(q, sq_b, sq_t, k, sk_b, sk_t, v, sv_b, sv_t, g, beta, s_in,
                                                    s_in_stride, s_out, s_out_stride, ids, inter, o, B, T, Hk, Hv,
                                                    scale, l2norm, din, nin, src, stream);
}

// v-split: more workgroups when there are few (b, h) tiles, so the launch
// still covers the 256 CUs with enough bytes in flight
static int recurrent_nvb(int B, int Hv) {
  const int64_t heads = static_cast<int64_t>(B) * Hv;
  return heads >= 2048 ? 1 : (heads >= 512 ? 2 : 4);
}

}  // namespace

extern "C" int gdn_recurrent(const uint16_t* q, int64_t sq_b, int64_t sq_t, const uint16_t* k,
                             int64_t sk_b, int64_t sk_t, const uint16_t* v, int64_t sv_b,
                             int64_t sv_t, const float* g, const uint16_t* beta,
                             const float* s_in, int64_t s_in_stride, float* s_out,
                             int64_t s_out_stride, const int64_t* ids, float* inter, uint16_t* o,
                             int B, int T, int Hk, int Hv, int D, float scale, int l2norm,
                             const float* src_states, const int64_t* src_accepted, int src_T, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (B < 0 || T < 1 || Hk <= 0 || Hv <= 0 || Hv % Hk) return GDN_ERR_INVALID_ARG;
  if (B == 0) return GDN_OK;
  if (!q || !k || !v || !g || !beta || !s_in || !o) return GDN_ERR_INVALID_ARG;
  if ((src_accepted != nullptr) != (src_states != nullptr) ||
      (src_states && (reinterpret_cast<uintptr_t>(src_states) % 16 || src_T < 1)))
    return GDN_ERR_INVALID_ARG;
  // float4 state access and 8-byte v access
  // a slot holds all Hv states (D x D, dense); a shorter slot stride would
  // make neighbouring slots overlap
  const int64_t slot_elems = static_cast<int64_t>(Hv) * D * D;
  const bool rows_distinct = ids || B > 1;
  if (rows_distinct && (s_in_stride < slot_elems || (s_out && s_out_stride < slot_elems))) return GDN_ERR_INVALID_ARG;
  if (s_in_stride % 4 || (s_out && s_out_stride % 4) || sv_b % 4 || sv_t % 4 ||
      reinterpret_cast<uintptr_t>(s_in) % 16 || (s_out && reinterpret_cast<uintptr_t>(s_out) % 16) ||
      (inter && reinterpret_cast<uintptr_t>(inter) % 16) || reinterpret_cast<uintptr_t>(v) % 8 ||
      reinterpret_cast<uintptr_t>(o) % 8)
    return GDN_ERR_INVALID_ARG;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nvb = recurrent_nvb(B, Hv);
  const DecodeIn din{};
  const NormIn nin{};
  const SrcIn src{src_states, src_accepted, src_T};
#define GDN_REC_ARGS q, sq_b, sq_t, k, sk_b, sk_t, v, sv_b, sv_t, g, beta, s_in, s_in_stride, s_out, \
                     s_out_stride, ids, inter, o, B, T, Hk, Hv, scale, l2norm, din, nin, src, s
  if (D == 128) {
    if (nvb == 1) return launch_recurrent<128, 1, 8>(GDN_REC_ARGS);
    if (nvb == 2) return launch_recurrent<128, 2>(GDN_REC_ARGS);
    return launch_recurrent<128, 4>(GDN_REC_ARGS);
  }
  if (nvb == 1) return launch_recurrent<64, 1>(GDN_REC_ARGS);
  if (nvb == 2) return launch_recurrent<64, 2>(GDN_REC_ARGS);
  return launch_recurrent<64, 4>(GDN_REC_ARGS);
#undef GDN_REC_ARGS
}

extern "C" int gdn_state_commit(float* pool, int64_t slot_stride, const int64_t* ids,
                                const float* inter, const int32_t* accepted, int B, int T, int Hv,
                                int D, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (B < 0 || T < 1 || Hv <= 0 || slot_stride % 4 || slot_stride < static_cast<int64_t>(Hv) * D * D)
    return GDN_ERR_INVALID_ARG;
  if (B == 0) return GDN_OK;
  if (!pool || !ids || !inter || !accepted) return GDN_ERR_INVALID_ARG;
  state_commit_kernel<<<dim3(static_cast<unsigned>(B * Hv)), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      pool, slot_stride, ids, inter, accepted, T, Hv, D);
  return gdn_launch_status();
}

extern "C" int gdn_recurrent_decode_fused(const uint16_t* q, int64_t sq_b, const uint16_t* k, int64_t sk_b,
                                          const uint16_t* x, int64_t sx_row, uint16_t* conv_pool,
                                          int64_t cp_slot, int64_t cp_ch, const uint16_t* conv_w,
                                          const uint16_t* a, const uint16_t* b, const void* A_log,
                                          const void* dt_bias, int param_is_fp32, float* s_pool,
                                          int64_t s_stride, const int64_t* ids, uint16_t* o, int B, int Hk,
                                          int Hv, int D, float scale, int l2norm, const uint16_t* z, int64_t sz_b,
                                          const uint16_t* norm_w, float eps, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (B < 0 || Hk <= 0 || Hv <= 0 || Hv % Hk) return GDN_ERR_INVALID_ARG;
  if (B == 0) return GDN_OK;
  if (!x || !conv_pool || !conv_w || !a || !b || !A_log || !dt_bias || !s_pool || !ids || !o)
    return GDN_ERR_INVALID_ARG;
  // q == k == NULL: their conv in the kernel as well (one key head per value head)
  const bool qk_fused = !q && !k;
  if ((!q || !k) && !(qk_fused && Hk == Hv)) return GDN_ERR_INVALID_ARG;
  const int64_t vbase = 2LL * Hk * D;  // first v channel of a raw row
  // float4 state access; 8-byte raw v and 16-byte tap reads
  if (s_stride % 4 || reinterpret_cast<uintptr_t>(s_pool) % 16 || sx_row % 4 ||
      sx_row < vbase + static_cast<int64_t>(Hv) * D || s_stride < static_cast<int64_t>(Hv) * D * D ||
      reinterpret_cast<uintptr_t>(x) % 8 || reinterpret_cast<uintptr_t>(conv_w) % 16 ||
      reinterpret_cast<uintptr_t>(o) % 8 || cp_ch < 3 || cp_slot < (vbase + static_cast<int64_t>(Hv) * D) * cp_ch)
    return GDN_ERR_INVALID_ARG;
  // the fused norm reads 8-byte pieces of z and of its weight
  if (z && (!norm_w || sz_b % 4 || sz_b < static_cast<int64_t>(Hv) * D || reinterpret_cast<uintptr_t>(z) % 8 ||
            reinterpret_cast<uintptr_t>(norm_w) % 8))
    return GDN_ERR_INVALID_ARG;
  const DecodeIn din{x + vbase,
                     sx_row,
                     conv_pool + vbase * cp_ch,
                     cp_slot,
                     cp_ch,
                     conv_w + vbase * 4,
                     a,
                     b,
                     A_log,
                     dt_bias,
                     param_is_fp32 ? 1 : 0,
                     qk_fused ? x : nullptr,
                     conv_pool,
                     conv_w,
                     Hk * D};
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the norm, and the q/k conv, need a head's D columns in one workgroup
  const int nvb = z || qk_fused ? 1 : recurrent_nvb(B, Hv);
  const NormIn nin{z, sz_b, norm_w, eps};
  const SrcIn src{};
#define GDN_REC_ARGS q, sq_b, 0, k, sk_b, 0, nullptr, 0, 0, nullptr, nullptr, s_pool, s_stride, s_pool, s_stride, \
                     ids, nullptr, o, B, 1, Hk, Hv, scale, l2norm, din, nin, src, s
  if (D == 128) {
    if (nvb == 1) return launch_recurrent<128, 1, 8>(GDN_REC_ARGS);
    if (nvb == 2) return launch_recurrent<128, 2>(GDN_REC_ARGS);
    return launch_recurrent<128, 4>(GDN_REC_ARGS);
  }
  if (nvb == 1) return launch_recurrent<64, 1>(GDN_REC_ARGS);
  if (nvb == 2) return launch_recurrent<64, 2>(GDN_REC_ARGS);
  return launch_recurrent<64, 4>(GDN_REC_ARGS);
#undef GDN_REC_ARGS
}

static int state_tile_pass(const float* src, float* dst, int64_t slot_stride, const int64_t* ids, int B, int Hv,
                           int D, void* stream) {
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (B < 0 || Hv <= 0 || slot_stride % 4 || slot_stride < static_cast<int64_t>(Hv) * D * D) return GDN_ERR_INVALID_ARG;
  if (B == 0) return GDN_OK;
  if (!src || !dst || !ids || reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return GDN_ERR_INVALID_ARG;
  const int64_t work = static_cast<int64_t>(B) * Hv;
  const int64_t grid = gdn::kNumXcd * ((work + gdn::kNumXcd - 1) / gdn::kNumXcd);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) {
    state_tile_pass_kernel<128, 512><<<dim3(static_cast<unsigned>(grid)), dim3(512), 0, s>>>(src, dst, slot_stride,
                                                                                            ids, B, Hv);
  } else {
    state_tile_pass_kernel<64, 256><<<dim3(static_cast<unsigned>(grid)), dim3(256), 0, s>>>(src, dst, slot_stride,
                                                                                           ids, B, Hv);
  }
  return gdn_launch_status();
}

extern "C" int gdn_state_tile_pass(float* pool, int64_t slot_stride, const int64_t* ids, int B, int Hv, int D,
                                   void* stream) {
  return state_tile_pass(pool, pool, slot_stride, ids, B, Hv, D, stream);
}

extern "C" int gdn_state_tile_copy(const float* src, float* dst, int64_t slot_stride, const int64_t* ids, int B,
                                   int Hv, int D, void* stream) {
  return state_tile_pass(src, dst, slot_stride, ids, B, Hv, D, stream);
}
