// The GDN layer's projections: C = A B^T on the bf16 matrix cores with fp32
// accumulation (F.linear with an nn.Linear weight, nanovllm/layers/linear.py:56-75,
// :133-158; called at nanovllm/models/qwen3_5.py:929-939, :964, :1008-1010,
// :1086).
//
//   A [M, K] bf16, row stride lda (activations: tokens x hidden, or the gated
//     norm's output for out_proj)
//   B [N, K] bf16, row stride ldb (the weight as nn.Linear stores it)
//   C [M, N] bf16, row stride ldc
//
// Both operands are K-contiguous, which is the layout the matrix-core
// fragments want: a 32x32x16 bf16 product takes from each lane 8 consecutive
// k values of one row of A (lane % 32) and of one row of B, so every operand
// read is one 16-byte LDS read.
//
// Tiling: a workgroup of 8 waves computes a BM x 256 tile of C (BM = 256, or
// 192 where that fills the last wave of tiles better), K in steps of 64.  Per
// step the A and B tiles (BM and 256 rows of 128 bytes) go global -> registers
// -> LDS, double-buffered (128 KiB of LDS at BM = 256): the loads of step s + 1
// are issued before the products of step s and written to the other buffer
// after them, one workgroup barrier per step.  Wave w owns rows BM / 2 (w / 4)
// .. + BM / 2 - 1 and columns 64 (w % 4) .. + 63: BM / 64 x 2 accumulator tiles
// of 32 x 32 (at BM = 256: 128 fp32 registers, 32 products per step).  LDS rows are 128 bytes with their eight
// 16-byte granules XOR-swizzled by (row % 8), so the 8 lanes of each LDS read
// phase hit 8 distinct granules (all 32 banks).
//
// Tile order: consecutive workgroups run on different XCDs (workgroup b on
// XCD b % 8); the tiles are renumbered so that each XCD walks a contiguous
// range in groups of 4 row blocks x all column blocks, and the tiles resident
// on one XCD at a time share A row blocks and B column blocks in its L2.
//
// Epilogue: the accumulators are rounded to bf16 and staged through LDS so
// each row goes out in 16-byte pieces.  With gate outputs (GemmGates) the
// columns [gate_col, gate_col + Hv) are the b projection and [gate_col + Hv,
// gate_col + 2 Hv) the a projection: besides their bf16 values, beta =
// sigmoid(b) (bf16) and g = -exp(A_log) softplus(a + dt_bias) (fp32) are
// written from the bf16-rounded values with the gate kernel's arithmetic
// (gdn::gate_beta, gdn::gate_g), so they equal gdn_g_beta applied to C.
#include "gdn_common.h"

namespace {

constexpr int kBN = 256, kBK = 64;  // row tile BM is a template argument: 256 or 192
constexpr int kGemmThreads = 512;
constexpr int kGroupM = 4;  // row blocks per tile group
constexpr int kCUs = 256;   // MI355X compute units: 8 XCDs x 32

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct GemmGates {
  float* g;               // [M, Hv] fp32 (NULL: no gate outputs)
  uint16_t* beta;         // [M, Hv] bf16
  const void* A_log;      // [Hv], bf16 or fp32 (param_f32)
  const void* dt_bias;
  int param_f32;
  int gate_col;           // first b column of C
  int Hv;
};

// byte offset of granule c (16 bytes) of row r in a 128-byte-row LDS tile
__device__ __forceinline__ int sw_off(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

__device__ __forceinline__ f32x16_t mfma_bf16(const gdn::s16x8_t& a, const gdn::s16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gdn::bf16x8_t, a),
                                                 __builtin_bit_cast(gdn::bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), 0x7fffffff, 0x00020000);
}

// Global -> register loads of one K step: 4 granules of A and 4 of B per
// thread; granule id = tid + 512 j: row id / 8, granule id % 8 (8 lanes per
// 128-byte row).  Rows past M (N) re-read the last row; their results are
// not stored.
template <int MI>
struct StepRegs {
  u32x4_t a[MI], b[4];
};

template <int MI>
__device__ __forceinline__ void load_step(StepRegs<MI>& R, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                          const int (&aoff)[MI], const int (&boff)[4], int kbyte) {
#pragma unroll
  for (int j = 0; j < MI; ++j) R.a[j] = __builtin_amdgcn_raw_buffer_load_b128(ra, aoff[j], kbyte, 0);
#pragma unroll
  for (int j = 0; j < 4; ++j) R.b[j] = __builtin_amdgcn_raw_buffer_load_b128(rb, boff[j], kbyte, 0);
}

template <int MI>
__device__ __forceinline__ void store_step(const StepRegs<MI>& R, uint8_t* la, uint8_t* lb, int tid) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int id = tid + kGemmThreads * j;
    const int off = sw_off(id >> 3, id & 7);
    if (j < MI) *reinterpret_cast<u32x4_t*>(la + off) = R.a[j];
    *reinterpret_cast<u32x4_t*>(lb + off) = R.b[j];
  }
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// grid = 8 * ceil(tiles / 8); block = 512.  BM / 64 granules of A per thread
// per step (MI), MI x 2 accumulator tiles per wave.
template <int BM>
__global__ __launch_bounds__(kGemmThreads, 1) void gemm_tn_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                                   const uint16_t* __restrict__ B, int64_t ldb,
                                                                   uint16_t* __restrict__ C, int64_t ldc, int M,
                                                                   int N, int K, GemmGates gt) {
  constexpr int MI = BM / 64;
  // 2 stages x (A, B) tiles of BM and 256 rows x 128 bytes (128 KiB for BM =
  // 256, 112 KiB for 192); the epilogue reuses it as one [BM][256] bf16 tile
  __shared__ __align__(16) uint8_t smem[2 * (BM + kBN) * 128];
  // stage s: A tile at s * (BM + 256) * 128 bytes, B tile BM * 128 bytes after it
  auto lds_a = [&](int st) { return smem + st * (BM + kBN) * 128; };
  auto lds_b = [&](int st) { return smem + st * (BM + kBN) * 128 + BM * 128; };

  const int mb_n = (M + BM - 1) / BM, nb_n = (N + kBN - 1) / kBN;
  const int64_t tiles = static_cast<int64_t>(mb_n) * nb_n;
  const int64_t L = gdn::xcd_remap(blockIdx.x, tiles);
  if (L < 0) return;
  // tile groups of kGroupM row blocks x all column blocks, row block fastest
  const int64_t per_group = static_cast<int64_t>(kGroupM) * nb_n;
  const int64_t grp = L / per_group, in_grp = L % per_group;
  const int gm = static_cast<int>(min<int64_t>(kGroupM, mb_n - grp * kGroupM));
  const int mb = static_cast<int>(grp * kGroupM + in_grp % gm);
  const int nb = static_cast<int>(in_grp / gm);
  const int m0 = mb * BM, n0 = nb * kBN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int li = lane & 31, lg = lane >> 5;

  // per-thread global byte offsets of its MI + 4 granules (row clamped)
  const __amdgpu_buffer_rsrc_t ra = rsrc_of(A), rb = rsrc_of(B);
  int aoff[MI], boff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int id = tid + kGemmThreads * j;
    const int r = id >> 3, c = id & 7;
    if (j < MI) aoff[j] = static_cast<int>((min(m0 + r, M - 1) * lda + 8 * c) * 2);
    boff[j] = static_cast<int>((min(n0 + r, N - 1) * ldb + 8 * c) * 2);
  }

  f32x16_t acc[MI][2];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = zero16();

  // Step s's tiles are loaded into register set s % 2 two steps ahead (so a
  // load has two steps of products to arrive), written to LDS buffer s % 2
  // at the end of step s - 1, and read there in step s.  Every path issues
  // the same loads (indices past the last step repeat it) so the compiler's
  // load counters stay exact; the loop runs two steps per trip.
  const int nk = K / kBK;
  auto products = [&](const uint8_t* la, const uint8_t* lb) {
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      gdn::s16x8_t af[MI], bf[2];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        af[i] = *reinterpret_cast<const gdn::s16x8_t*>(la + sw_off((BM / 2) * wm + 32 * i + li, 2 * ks + lg));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        bf[j] = *reinterpret_cast<const gdn::s16x8_t*>(lb + sw_off(64 * wn + 32 * j + li, 2 * ks + lg));
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(af[i], bf[j], acc[i][j]);
    }
  };
  auto kb = [&](int st) { return min(st, nk - 1) * kBK * 2; };
  StepRegs<MI> R0, R1;
  load_step(R0, ra, rb, aoff, boff, kb(0));
  gdn::keep_loads_here();
  load_step(R1, ra, rb, aoff, boff, kb(1));
  gdn::keep_loads_here();
  store_step(R0, lds_a(0), lds_b(0), tid);
  gdn::lds_barrier();
  int s = 0;
  for (; s + 1 < nk; s += 2) {
    load_step(R0, ra, rb, aoff, boff, kb(s + 2));     // step s + 2 (set 0 was written out)
    gdn::keep_loads_here();
    products(lds_a(0), lds_b(0));                      // step s
    store_step(R1, lds_a(1), lds_b(1), tid);           // step s + 1
    gdn::lds_barrier();
    load_step(R1, ra, rb, aoff, boff, kb(s + 3));     // step s + 3
    gdn::keep_loads_here();
    products(lds_a(1), lds_b(1));                      // step s + 1
    if (s + 2 < nk) store_step(R0, lds_a(0), lds_b(0), tid);  // step s + 2
    gdn::lds_barrier();
  }
  if (s < nk) products(lds_a(0), lds_b(0));            // the last step when nk is odd
  __syncthreads();  // the staged tile reuses the buffers; no loads left to keep in flight

  // ---- epilogue: bf16 tile through LDS, 16-byte row pieces out ----
  // wave (wm, wn) stages its BM / 2 x 64 tile at rows BM / 2 wm .., columns
  // 64 wn .. of a [BM][256] bf16 tile (512-byte rows, granules swizzled by row % 32)
  uint16_t* ct = reinterpret_cast<uint16_t*>(smem);
  auto c_off = [](int r, int c8) { return r * 256 + (((c8) ^ (r & 31)) << 3); };
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = 64 * wn + 32 * j + li;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = (BM / 2) * wm + 32 * i + 8 * q + 4 * lg + r;
          ct[c_off(row, col >> 3) + (col & 7)] = gdn::f2bf(acc[i][j][4 * q + r]);
        }
    }
  gdn::lds_barrier();
  // BM rows x 32 granules, BM / 16 per thread
#pragma unroll 4
  for (int e = tid; e < BM * (kBN / 8); e += kGemmThreads) {
    const int row = e >> 5, c8 = e & 31;
    const int m = m0 + row, n = n0 + 8 * c8;
    if (m >= M || n >= N) continue;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(ct + c_off(row, c8));
    uint16_t* cp = C + static_cast<int64_t>(m) * ldc + n;
    if (n + 8 <= N && ldc % 8 == 0) {
      *reinterpret_cast<u32x4_t*>(cp) = v;
    } else {
      const uint16_t* vs = reinterpret_cast<const uint16_t*>(&v);
      for (int t = 0; t < min(8, N - n); ++t) cp[t] = vs[t];
    }
    if (gt.g && n + 8 > gt.gate_col && n < gt.gate_col + 2 * gt.Hv) {
      const uint16_t* vs = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const int col = n + t - gt.gate_col;
        if (col < 0 || col >= 2 * gt.Hv || n + t >= N) continue;
        if (col < gt.Hv) {
          gt.beta[static_cast<int64_t>(m) * gt.Hv + col] = gdn::gate_beta(gdn::bf2f(vs[t]));
        } else {
          const int h = col - gt.Hv;
          gt.g[static_cast<int64_t>(m) * gt.Hv + h] =
              gdn::gate_g(gdn::bf2f(vs[t]), gdn::load_param(gt.A_log, h, gt.param_f32),
                          gdn::load_param(gt.dt_bias, h, gt.param_f32));
        }
      }
    }
  }
}

}  // namespace

extern "C" int gdn_gemm_bf16(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, uint16_t* C,
                             int64_t ldc, int M, int N, int K, float* g, uint16_t* beta, const void* A_log,
                             const void* dt_bias, int param_is_fp32, int gate_col, int Hv, void* stream) {
  if (M < 0 || N < 0 || K < 0) return GDN_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return GDN_OK;
  if (!A || !B || !C) return GDN_ERR_INVALID_ARG;
  // K in steps of 64; 16-byte row pieces of A, B and C; 32-bit buffer offsets
  // (C rows whose stride is not a multiple of 8 go out element by element)
  if (K % kBK || K == 0 || lda % 8 || ldb % 8 || lda < K || ldb < K || ldc < N ||
      reinterpret_cast<uintptr_t>(A) % 16 || reinterpret_cast<uintptr_t>(B) % 16 ||
      reinterpret_cast<uintptr_t>(C) % (ldc % 8 ? 2 : 16) || static_cast<int64_t>(M) * lda * 2 >= (1LL << 31) ||
      static_cast<int64_t>(N) * ldb * 2 >= (1LL << 31))
    return GDN_ERR_INVALID_ARG;
  if (g && (!beta || !A_log || !dt_bias || Hv <= 0 || gate_col < 0 || gate_col + 2 * Hv > N)) return GDN_ERR_INVALID_ARG;
  const GemmGates gt{g, beta, A_log, dt_bias, param_is_fp32 ? 1 : 0, gate_col, Hv};
  // Row tile: one workgroup per CU, so a launch runs in ceil(tiles / CUs)
  // waves of tiles, each taking time in proportion to the tile's rows.  The
  // 192-row tile is taken when its waves x rows is smaller (a short last
  // wave of 256-row tiles, e.g. 536 tiles = 2.09 waves -> 712 = 2.78).
  const int64_t nbn = (N + kBN - 1) / kBN;
  const int64_t t256 = ((M + 255) / 256) * nbn, t192 = ((M + 191) / 192) * nbn;
  const int64_t w256 = (t256 + kCUs - 1) / kCUs, w192 = (t192 + kCUs - 1) / kCUs;
  const bool small = w192 * 192 < w256 * 256;
  const int64_t tiles = small ? t192 : t256;
  const int64_t grid = gdn::kNumXcd * ((tiles + gdn::kNumXcd - 1) / gdn::kNumXcd);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (small)
    gemm_tn_kernel<192><<<dim3(static_cast<unsigned>(grid)), dim3(kGemmThreads), 0, st>>>(A, lda, B, ldb, C, ldc,
                                                                                         M, N, K, gt);
  else
    gemm_tn_kernel<256><<<dim3(static_cast<unsigned>(grid)), dim3(kGemmThreads), 0, st>>>(A, lda, B, ldb, C, ldc,
                                                                                         M, N, K, gt);
  return gdn_launch_status();
}
