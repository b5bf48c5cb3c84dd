// Gated RMSNorm over the value head dim (D = 64 or 128), rounding in the
// eager order of nanovllm/models/qwen3_5.py:121-131:
//   n  = bf16(x * rsqrt(mean(x^2) + eps))      (fp32 math)
//   wn = bf16(w * n)                           (bf16 x bf16 product)
//   y  = bf16(float(wn) * silu(float(z)))
// 3 * D * 2 bytes per row, but bound by the vector ALUs in practice: the
// exact SiLU is most of the ~30 instructions per element.  D/8 lanes per
// row, 16-byte vectors.
#include "gdn_common.h"

namespace {

template <int D>
__global__ __launch_bounds__(256) void rmsnorm_gated_kernel(const uint16_t* __restrict__ x,
                                                            int64_t sx_tok,
                                                            const uint16_t* __restrict__ z,
                                                            int64_t sz_tok,
                                                            const uint16_t* __restrict__ w,
                                                            uint16_t* __restrict__ y,
                                                            int64_t n_sel, int H, float eps,
                                                            const int64_t* __restrict__ ranges, int n_ranges,
                                                            int64_t n_tok) {
  // block b = kRowsPerBlock consecutive selected tokens (block b / H) of head
  // b % H: the division is the block's, in scalar registers, and the H blocks
  // of a token block run side by side over one contiguous stretch of rows
  constexpr int kLanes = D / 8;                 // lanes per row
  constexpr int kRowsPerBlock = 256 / kLanes;
  const int lane = threadIdx.x % kLanes;
  const uint32_t b = blockIdx.x;
  const int h = static_cast<int>(b % static_cast<uint32_t>(H));
  const int64_t t_sel = static_cast<int64_t>(b / static_cast<uint32_t>(H)) * kRowsPerBlock + threadIdx.x / kLanes;
  bool active = t_sel < n_sel;
  int64_t tok = active ? t_sel : 0;
  if (ranges && active) {
    // token ranges (start, count, tokens before it): the t-th selected token;
    // a token that no range holds, or that falls outside the n_tok rows, is
    // skipped
    bool found = false;
    for (int i = 0; i < n_ranges; ++i) {
      const int64_t start = ranges[3 * i], cnt = ranges[3 * i + 1], before = ranges[3 * i + 2];
      if (tok >= before && tok < before + cnt) {
        tok = start + (tok - before);
        found = true;
        break;
      }
    }
    active = found && tok >= 0 && tok < n_tok;
    if (!active) tok = 0;
  }
  const int64_t row = tok * H + h;

  uint4 xv = make_uint4(0, 0, 0, 0), zv = make_uint4(0, 0, 0, 0);
  if (active) {
    xv = *reinterpret_cast<const uint4*>(x + tok * sx_tok + static_cast<int64_t>(h) * D + lane * 8);
    zv = *reinterpret_cast<const uint4*>(z + tok * sz_tok + static_cast<int64_t>(h) * D + lane * 8);
  }
  const uint4 wv = *reinterpret_cast<const uint4*>(w + lane * 8);
  const uint16_t* xs = reinterpret_cast<const uint16_t*>(&xv);
  const uint16_t* zs = reinterpret_cast<const uint16_t*>(&zv);
  const uint16_t* ws = reinterpret_cast<const uint16_t*>(&wv);

  float xf[8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xf[i] = gdn::bf2f(xs[i]);
    ss += xf[i] * xf[i];
  }
#pragma unroll
  for (int m = kLanes / 2; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  const float r = rsqrtf(ss / static_cast<float>(D) + eps);

  // (the conv's exp2 + reciprocal form of silu is 10 % faster here but moves
  // about 3 in 10^4 outputs by one bf16 ulp: on outputs above 8 that is more
  // than the 2e-2 max-abs bar)
  float yv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) yv[i] = gdn::norm_gate(xf[i], r, gdn::bf2f(ws[i]), gdn::bf2f(zs[i]));
  uint4 out;
  out.x = gdn::f2bf2(yv[0], yv[1]);
  out.y = gdn::f2bf2(yv[2], yv[3]);
  out.z = gdn::f2bf2(yv[4], yv[5]);
  out.w = gdn::f2bf2(yv[6], yv[7]);
  if (active) *reinterpret_cast<uint4*>(y + row * D + lane * 8) = out;  // y rows [tok, h] dense
}

}  // namespace

extern "C" int gdn_rmsnorm_gated(const uint16_t* x, int64_t sx_tok, const uint16_t* z,
                                 int64_t sz_tok, const uint16_t* w, uint16_t* y, int64_t n_tok,
                                 int H, int D, float eps, void* stream) {
  if (n_tok < 0 || H <= 0) return GDN_ERR_INVALID_ARG;
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (n_tok == 0) return GDN_OK;
  if (!x || !z || !w || !y) return GDN_ERR_INVALID_ARG;
  // 16-byte vector access needs 8-element alignment of every row start.
  if ((sx_tok % 8) || (sz_tok % 8) || (reinterpret_cast<uintptr_t>(x) % 16) ||
      (reinterpret_cast<uintptr_t>(z) % 16) || (reinterpret_cast<uintptr_t>(w) % 16) ||
      (reinterpret_cast<uintptr_t>(y) % 16))
    return GDN_ERR_INVALID_ARG;
  if ((n_tok + 15) / 16 * H >= (1LL << 32)) return GDN_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) {
    const int64_t nb = (n_tok + 15) / 16;
    rmsnorm_gated_kernel<128><<<dim3(static_cast<unsigned>(nb * H)), dim3(256), 0, s>>>(x, sx_tok, z, sz_tok, w, y, n_tok,
                                                                                        H, eps, nullptr, 0, n_tok);
  } else {
    const int64_t nb = (n_tok + 31) / 32;
    rmsnorm_gated_kernel<64><<<dim3(static_cast<unsigned>(nb * H)), dim3(256), 0, s>>>(x, sx_tok, z, sz_tok, w, y, n_tok,
                                                                                       H, eps, nullptr, 0, n_tok);
  }
  return gdn_launch_status();
}

extern "C" int gdn_rmsnorm_gated_ranges(const uint16_t* x, int64_t sx_tok, const uint16_t* z, int64_t sz_tok,
                                        const uint16_t* w, uint16_t* y, int64_t n_tok, const int64_t* ranges,
                                        int n_ranges, int64_t n_sel_tok, int H, int D, float eps, void* stream) {
  if (n_sel_tok < 0 || n_tok < 0 || n_sel_tok > n_tok || H <= 0 || n_ranges < 0) return GDN_ERR_INVALID_ARG;
  if (D != 64 && D != 128) return GDN_ERR_UNSUPPORTED;
  if (n_sel_tok == 0) return GDN_OK;
  if (!x || !z || !w || !y || !ranges || n_ranges == 0) return GDN_ERR_INVALID_ARG;
  if ((sx_tok % 8) || (sz_tok % 8) || (reinterpret_cast<uintptr_t>(x) % 16) ||
      (reinterpret_cast<uintptr_t>(z) % 16) || (reinterpret_cast<uintptr_t>(w) % 16) ||
      (reinterpret_cast<uintptr_t>(y) % 16))
    return GDN_ERR_INVALID_ARG;
  if ((n_sel_tok + 15) / 16 * H >= (1LL << 32)) return GDN_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (D == 128) {
    const int64_t nb = (n_sel_tok + 15) / 16;
    rmsnorm_gated_kernel<128><<<dim3(static_cast<unsigned>(nb * H)), dim3(256), 0, s>>>(
        x, sx_tok, z, sz_tok, w, y, n_sel_tok, H, eps, ranges, n_ranges, n_tok);
  } else {
    const int64_t nb = (n_sel_tok + 31) / 32;
    rmsnorm_gated_kernel<64><<<dim3(static_cast<unsigned>(nb * H)), dim3(256), 0, s>>>(
        x, sx_tok, z, sz_tok, w, y, n_sel_tok, H, eps, ranges, n_ranges, n_tok);
  }
  return gdn_launch_status();
}
