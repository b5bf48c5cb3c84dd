// Fused gate / beta:  g = -exp(A_log) * softplus(a + dt_bias)  (fp32),
//                     beta = sigmoid(b)                          (bf16).
// Follows nanovllm/models/qwen3_5.py:320-342 (softplus threshold 20, g = 0 on
// masked padding rows).  Pure elementwise, HBM-bound: 2+2 bytes in, 4+2 out
// per element, one thread per element.
#include "gdn_common.h"

namespace {

template <bool kParamF32>
__device__ __forceinline__ float load_param(const void* p, int h) {
  if constexpr (kParamF32) return static_cast<const float*>(p)[h];
  else return gdn::bf2f(static_cast<const uint16_t*>(p)[h]);
}

template <bool kParamF32, bool kHasMask>
__global__ __launch_bounds__(256) void g_beta_kernel(const uint16_t* __restrict__ b,
                                                     const uint16_t* __restrict__ a,
                                                     const void* __restrict__ A_log,
                                                     const void* __restrict__ dt_bias,
                                                     const uint8_t* __restrict__ mask,
                                                     float* __restrict__ g,
                                                     uint16_t* __restrict__ beta, int64_t total,
                                                     int Hv) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int h = static_cast<int>(i % Hv);
  const float av = gdn::bf2f(a[i]);
  const float bv = gdn::bf2f(b[i]);
  const float al = load_param<kParamF32>(A_log, h);
  const float dt = load_param<kParamF32>(dt_bias, h);
  float gv = gdn::gate_g(av, al, dt);
  if constexpr (kHasMask) {
    if (mask[i / Hv] == 0) gv = 0.0f;
  }
  g[i] = gv;
  beta[i] = gdn::gate_beta(bv);
}

}  // namespace

extern "C" int gdn_g_beta(const uint16_t* b, const uint16_t* a, const void* A_log,
                          const void* dt_bias, int param_is_fp32, const uint8_t* mask, float* g,
                          uint16_t* beta, int64_t total, int Hv, void* stream) {
  if (total < 0 || Hv <= 0 || total % Hv != 0) return GDN_ERR_INVALID_ARG;
  if (total == 0) return GDN_OK;
  if (!b || !a || !A_log || !dt_bias || !g || !beta) return GDN_ERR_INVALID_ARG;
  const dim3 block(256);
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (param_is_fp32) {
    if (mask) g_beta_kernel<true, true><<<grid, block, 0, s>>>(b, a, A_log, dt_bias, mask, g, beta, total, Hv);
    else g_beta_kernel<true, false><<<grid, block, 0, s>>>(b, a, A_log, dt_bias, mask, g, beta, total, Hv);
  } else {
    if (mask) g_beta_kernel<false, true><<<grid, block, 0, s>>>(b, a, A_log, dt_bias, mask, g, beta, total, Hv);
    else g_beta_kernel<false, false><<<grid, block, 0, s>>>(b, a, A_log, dt_bias, mask, g, beta, total, Hv);
  }
  return gdn_launch_status();
}

extern "C" int gdn_abi_version(void) { return GDN_ABI_VERSION; }
