// Shared device helpers for the gfx950 GDN kernels: bf16 bit conversions,
// MFMA fragment types, wave reductions, XCD-aware block remapping and the
// launch-status plumbing used by every extern "C" entry point.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gdn_mi355x.h"

namespace gdn {

// ---- bf16 <-> fp32 ----
// float -> bf16 uses the gfx950 hardware conversion (v_cvt_pk_bf16_f32,
// round-to-nearest-even), which matches torch's rounding for every non-NaN
// value.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// two conversions in one instruction: low half = a, high half = b
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// hi/lo split of an fp32 value into two bf16 terms: x ~= hi + lo with
// |x - hi - lo| <= 2^-16 |x|.  Used to run fp32-accurate products on the
// bf16 matrix cores (two or three MFMA passes).
__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
  hi = f2bf(x);
  lo = f2bf(x - bf2f(hi));
}

// e^y through the hardware exp2 with the argument's rounding error put back:
// y log2(e) = t + err exactly up to ~2^-48 |y| (two-product and the low part
// of log2(e)), and 2^(t + err) = 2^t (1 + err ln 2) to second order.  A few
// ulp in fp32 for |y| < 88 (the hardware exp2 itself is within 1 ulp);
// overflow and underflow come out as inf and 0 like expf.
__device__ __forceinline__ float exp_acc(float y) {
  constexpr float kLog2e = 1.44269504088896340736f;       // rounded to fp32
  constexpr float kLog2eLo = 1.925963033500011e-08f;      // log2(e) - kLog2e
  constexpr float kLn2 = 0.69314718055994530942f;
  const float t = y * kLog2e;
  const float err = fmaf(y, kLog2e, -t) + y * kLog2eLo;
  const float p = __builtin_amdgcn_exp2f(t);
  return fmaf(p, err * kLn2, p);
}

// y = acc * sigmoid(acc), the reference conv epilogue's form (acc *
// tl.sigmoid(acc), which lowers to an exp2 of the scaled argument and a
// reciprocal): e^-acc as the hardware exp2 of -acc log2(e), then the hardware
// reciprocal of 1 + e^-acc.  Relative error <= ~1e-7 (|acc| + 2) -- the
// argument's rounding times log2(e) ln 2 plus an ulp each for exp2 and rcp --
// far below the bf16 output step (3.9e-3).  For acc < -88.7 e^-acc is +inf,
// its reciprocal 0 and y = -0, as the divide gives.
__device__ __forceinline__ float silu_acc(float acc) {
  const float e = __builtin_amdgcn_exp2f(acc * -1.44269504088896340736f);
  return acc * __builtin_amdgcn_rcpf(1.0f + e);
}

// Causal depthwise conv of width 4 at one channel (x0 the oldest input, x3 the
// current one; w the channel's 4 taps) followed by SiLU, in one fixed operation
// order: every varlen conv path (the standalone conv kernel, and the conv fused
// into the chunk kernels: q and k in the prep kernel, v in the state kernel's
// U waves) goes through this, so they agree bit for bit.
__device__ __forceinline__ float conv4_silu(float x0, float x1, float x2, float x3, const float* w) {
  float acc = x0 * w[0];
  acc = fmaf(x1, w[1], acc);
  acc = fmaf(x2, w[2], acc);
  acc = fmaf(x3, w[3], acc);
  return silu_acc(acc);
}

// Decode conv of one channel (one token): y = silu(x w[3] + s0 w[0] + s1 w[1] +
// s2 w[2]) in that accumulation order (the reference's decode epilogue), with
// s0 the oldest state tap.  Shared by the decode conv kernel and the fused
// decode step, so they agree bit for bit.
__device__ __forceinline__ float conv_decode_silu(float x, float s0, float s1, float s2, const float* w) {
  float acc = x * w[3];
  acc = fmaf(s0, w[0], acc);
  acc = fmaf(s1, w[1], acc);
  acc = fmaf(s2, w[2], acc);
  return silu_acc(acc);
}

// The reference writes the rolled conv state as (x + s) with the other operand
// masked to zero, which maps -0.0 to +0.0 and is otherwise a bit copy.
__device__ __forceinline__ uint16_t roll_value(uint16_t bits) {
  return bits == 0x8000u ? static_cast<uint16_t>(0) : bits;
}

// Gates of one (token, value head): g = -exp(A_log) * softplus(a + dt_bias)
// (softplus threshold 20) and beta = sigmoid(b) rounded to bf16, with libm's
// expf / logf.  Shared by the gate kernel and the fused chunk prep kernel.
__device__ __forceinline__ float gate_g(float a, float A_log, float dt_bias) {
  const float z = a + dt_bias;
  const float sp = z > 20.0f ? z : logf(1.0f + expf(z));
  return -expf(A_log) * sp;
}
__device__ __forceinline__ uint16_t gate_beta(float b) { return f2bf(1.0f / (1.0f + expf(-b))); }

// A per-head parameter stored as bf16 (is_f32 = 0) or fp32.
__device__ __forceinline__ float load_param(const void* p, int h, int is_f32) {
  return is_f32 ? static_cast<const float*>(p)[h] : bf2f(static_cast<const uint16_t*>(p)[h]);
}

// ---- MFMA fragment types (v_mfma_f32_16x16x32_bf16) ----
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16x16x32(const s16x8_t& a, const s16x8_t& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// fp32 matrix-core product, 16x16x4: A lane l = A[l&15][l>>4], B lane l = B[l>>4][l&15].
__device__ __forceinline__ f32x4_t mfma16x16x4f32(float a, float b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One element of the gated RMSNorm after the row's r = rsqrt(mean(x^2) + eps)
// (nanovllm/models/qwen3_5.py:121-131, eager rounding order):
//   n = bf16(x r), wn = bf16(w n), y = wn * silu(z)   (the caller rounds y)
// silu(z) = z / (1 + e^-z): e^-z within a few ulp (exp_acc) and the divide as
// a hardware reciprocal refined by one Newton step (within an ulp of the
// divide); the exponent is capped at 88 so the step never sees an infinite
// operand.  Every gated-norm output goes through this function, so the
// standalone and the fused norms agree bit for bit.
__device__ __forceinline__ float norm_gate(float x, float r, float w, float z) {
  const float n = bf2f(f2bf(x * r));
  const float wn = bf2f(f2bf(w * n));
  // (0 - z rather than -z: a subtraction's result needs no canonicalising
  // before the min; exp of +0 and -0 are the same)
  const float d = 1.0f + exp_acc(fminf(0.0f - z, 88.0f));
  float rc = __builtin_amdgcn_rcpf(d);
  rc = fmaf(rc, fmaf(-d, rc, 1.0f), rc);
  return wn * (z * rc);
}

// ---- wave-level reductions (wave64) ----
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// ---- workgroup barrier ordering LDS only ----
// __syncthreads() fences every address space, which on gfx950 waits for all
// outstanding global loads (vmcnt(0)) and so drains a software prefetch at
// each barrier.  This barrier orders LDS accesses only (lgkmcnt(0)); global
// loads stay in flight across it.  Global memory written by one wave and read
// by another still needs __syncthreads().
// Compiler-level fence for memory operations (emits no instruction): loads
// issued before it stay before it, so a prefetch is not sunk next to its use.
__device__ __forceinline__ void keep_loads_here() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ void lds_barrier() {
  // No instruction is scheduled across the barrier: work moved ahead of it
  // would wait there on loads that are meant to stay in flight.
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  __builtin_amdgcn_sched_barrier(0);
}

// ---- XCD-aware block remap ----
// Workgroups are dispatched round-robin over the 8 XCDs (block b lands on XCD
// b % 8).  Remapping gives each XCD a contiguous range of work items, so the
// blocks that share operands (e.g. the v-blocks of one head) share one L2.
// Launch with grid = 8 * ceil(total / 8); returns -1 for padding blocks.
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t total) {
  const int64_t per = (total + 7) / 8;
  const int64_t w = (b % 8) * per + b / 8;
  return w < total ? w : -1;
}

constexpr int kNumXcd = 8;
constexpr int kNumCu = 256;  // MI355X compute units: 8 XCDs x 32

}  // namespace gdn

// Status of the last launch on this thread, as an entry-point return code.
static inline int gdn_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? GDN_OK : static_cast<int>(e);
}
