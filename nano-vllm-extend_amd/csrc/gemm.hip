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
// k values of one row of each operand, so every operand read is one 16-byte
// LDS read.
//
// Tiling: a workgroup of 4 waves (one per SIMD, one workgroup per CU)
// computes a BM x 256 tile of C (BM = 256, or 192 where that fills the last
// wave of tiles better; 64 x 128 or 64 x 64, several workgroups per CU, for
// small M, with three or four LDS stages when K is long: gemm_tn_deep_kernel
// below), K in steps of 64.  Wave (wm, wn) owns rows BM / 2 wm
// .. and columns 128 wn ..: BM / 64 x 4 accumulator tiles of 32 x 32 (256
// registers at BM = 256, kept in AGPRs), 64 products per step.
//
// Operand path: global -> LDS directly (buffer_load ... lds, no registers),
// two stages of BM + 256 rows x 128 bytes (128 KiB at BM = 256).  The loads
// of step s + 1 are spread one per product over the first half of step s (a
// burst stalls the waves on the shared address unit).  Operand fragments
// are read one 16-deep sub-step ahead of their products, interleaved one read
// per product.  One workgroup barrier per step, placed before the last
// sub-step's products so the next stage's first reads overlap them.  LDS
// rows have their eight 16-byte granules XOR-swizzled by (row / 2) % 8, which
// makes the fragment reads free of bank conflicts (measured: zero).
//
// Tile order: consecutive workgroups run on different XCDs (workgroup b on
// XCD b % 8); the tiles are renumbered so that each XCD walks a contiguous
// range in groups of 4 row blocks x all column blocks, and the tiles resident
// on one XCD at a time share A row blocks and B column blocks in its L2.
//
// Epilogue: the products take B as the first operand, so they are tiles of
// C^T and each lane holds runs of 4 consecutive columns of one row; a lane
// swap (v_permlane32_swap) makes them runs of 8, stored as 16-byte pieces
// straight from the registers.  With gate outputs (GemmGates) the columns
// [gate_col, gate_col + Hv) are the b projection and [gate_col + Hv, gate_col
// + 2 Hv) the a projection: besides their bf16 values, beta = sigmoid(b)
// (bf16) and g = -exp(A_log) softplus(a + dt_bias) (fp32) are written from the
// bf16-rounded values with the gate kernel's arithmetic (gdn::gate_beta,
// gdn::gate_g), so they equal gdn_g_beta applied to C.
#include "gdn_common.h"

namespace {

constexpr int kBK = 64;  // the tile (BM x BN) is a template argument
constexpr int kGemmThreads = 256;
constexpr int kGroupM = 4;  // row blocks per tile group
constexpr int kCUs = gdn::kNumCu;

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// The output: C's columns in up to four parts, part s holding columns
// [end[s - 1], end[s]) (end[-1] = 0) at c[s] with row stride ld[s]; vec[s]: its
// rows take 16-byte stores.  Every part boundary is a multiple of 16, so each
// 16-column half of a 32-column block (one store pair of every lane) lies in
// one part, and the part is the same for the whole wave.
constexpr int kMaxParts = 4;
struct GemmOut {
  uint16_t* c[kMaxParts];
  int64_t ld[kMaxParts];
  int end[kMaxParts];
  int vec[kMaxParts];
};

struct GemmGates {
  float* g;               // [M, Hv] fp32 (NULL: no gate outputs)
  uint16_t* beta;         // [M, Hv] bf16
  const void* A_log;      // [Hv], bf16 or fp32 (param_f32)
  const void* dt_bias;
  int param_f32;
  int gate_col;           // first b column of C
  int Hv;
};

// Byte offset of granule c (16 bytes) of row r in a 128-byte-row LDS tile.
// Granules are XOR-swizzled by (r / 2) % 8: a 16-byte read serves 16 lanes
// at a time from 256 bytes of banks (two rows), and the 16 lanes of a
// fragment read (16 consecutive rows, one granule) then hit 16 distinct
// 16-byte bank groups.
__device__ __forceinline__ int sw_off(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

__device__ __forceinline__ f32x16_t mfma_bf16(const gdn::s16x8_t& a, const gdn::s16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gdn::bf16x8_t, a),
                                                 __builtin_bit_cast(gdn::bf16x8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), 0x7fffffff, 0x00020000);
}

// Direct-to-LDS loads: one buffer_load_dwordx4 ... lds moves 64 lanes x 16
// bytes into the 1 KiB of LDS at M0 + 16 lane.  A stage holds the A tile (BM
// rows) then the B tile (256 rows), 128 bytes a row: 1 KiB block b is tile rows
// 8 b' .. 8 b' + 7 (b' = b for A, b - BM / 8 for B; BM / 8 is even).  Lane l
// fills row 8 b' + l / 8, slot l % 8, which under the swizzle holds the row's
// global granule (l % 8) ^ (4 (b % 2) + l / 16).  Wave w loads blocks w,
// w + 4, w + 8, ...
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint8_t* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr_t)lds, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Epilogue of a BM x BN tile, straight from the accumulators of wave
// (wm, wn).  `scratch`: (BM / 2) x 32 bf16 per wave of LDS that nothing reads
// any more (the gate outputs go through it).
template <int BM, int BN>
__device__ __forceinline__ void gemm_store(const f32x16_t (&acc)[BM / 64][BN / 64], const GemmOut& out, int M,
                                           int N, int m0, int n0, int wave, int lane, const GemmGates& gt,
                                           uint8_t* scratch) {
  constexpr int MI = BM / 64, NJ = BN / 64;
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lg = lane >> 5;
  // acc[i][j] register 4 q + r of lane (li, lg) is C[row][col + r] with row =
  // m0 + BM / 2 wm + 32 i + li, col = n0 + BN / 2 wn + 32 j + 8 q + 4 lg.  One
  // swap between lanes l and l + 32 (v_permlane32_swap: the upper half of the
  // first operand with the lower half of the second) leaves lane (li, lg)
  // columns 16 p + 8 lg .. + 7 of pair p = (q 2p, q 2p + 1) in bf16: one
  // 16-byte store per pair, two lanes filling 32 bytes of a row.
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int m = m0 + (BM / 2) * wm + 32 * i + li;
    const bool row_ok = m < M;  // (no early exit: the gate loop below spans every lane)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int cb = n0 + (BN / 2) * wn + 32 * j;  // wave-uniform
      if (cb >= N) continue;
      // the output part of this block's first 16 columns (wave-uniform;
      // selects with constant indices, so the part table stays in scalar
      // registers)
      int s = cb < out.end[0] ? 0 : cb < out.end[1] ? 1 : cb < out.end[2] ? 2 : 3;
      auto pick = [&s](auto a0, auto a1, auto a2, auto a3) { return s == 0 ? a0 : s == 1 ? a1 : s == 2 ? a2 : a3; };
      int cbeg = pick(0, out.end[0], out.end[1], out.end[2]);
      int cend = pick(out.end[0], out.end[1], out.end[2], out.end[3]);
      bool vec = pick(out.vec[0], out.vec[1], out.vec[2], out.vec[3]) != 0;
      uint16_t* crow = pick(out.c[0], out.c[1], out.c[2], out.c[3]) +
                       static_cast<int64_t>(row_ok ? m : 0) * pick(out.ld[0], out.ld[1], out.ld[2], out.ld[3]) - cbeg;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (p == 1 && cend == cb + 16 && cend < N) {
          // the second 16 columns open the next part (a boundary inside the
          // block: rare)
          ++s;
          cbeg = cend;
          cend = pick(out.end[0], out.end[1], out.end[2], out.end[3]);
          vec = pick(out.vec[0], out.vec[1], out.vec[2], out.vec[3]) != 0;
          crow = pick(out.c[0], out.c[1], out.c[2], out.c[3]) +
                 static_cast<int64_t>(row_ok ? m : 0) * pick(out.ld[0], out.ld[1], out.ld[2], out.ld[3]) - cbeg;
        }
        const int q = 2 * p;
        const auto lo = __builtin_amdgcn_permlane32_swap(gdn::f2bf2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                                                         gdn::f2bf2(acc[i][j][4 * q + 4], acc[i][j][4 * q + 5]),
                                                         false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap(gdn::f2bf2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]),
                                                         gdn::f2bf2(acc[i][j][4 * q + 6], acc[i][j][4 * q + 7]),
                                                         false, false);
        const uint32_t w[4] = {lo[0], hi[0], lo[1], hi[1]};  // columns n .. n + 7
        const int n = cb + 16 * p + 8 * lg;
        if (!row_ok) {
        } else if (vec && n + 8 <= cend) {
          *reinterpret_cast<uint4*>(crow + n) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
#pragma unroll
          for (int t = 0; t < 8; ++t)
            if (n + t < cend) crow[n + t] = static_cast<uint16_t>(w[t / 2] >> (16 * (t % 2)));
        }
      }
      // Gate outputs from the bf16-rounded b and a columns of this 32-column
      // block.  The block's values go through the wave's own 8 KiB of the
      // stage the last step no longer reads (wave-local, in order), and a
      // rolled loop computes beta and g (unrolled over the registers, the gate
      // arithmetic would not fit beside the accumulators).
      if (gt.g && cb + 32 > gt.gate_col && cb < gt.gate_col + 2 * gt.Hv) {
        uint16_t* gs = reinterpret_cast<uint16_t*>(scratch) + wave * (BM / 2) * 32;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = gdn::f2bf2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
          const uint32_t hi = gdn::f2bf2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          *reinterpret_cast<uint2*>(gs + 32 * (32 * i + li) + 8 * q + 4 * lg) = make_uint2(lo, hi);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll 1
        for (int e = lane; e < 32 * 32; e += 64) {
          const int r = e >> 5, c = e & 31;
          const int mm = m - li + r, n = cb + c, col = n - gt.gate_col;
          if (mm >= M || n >= N || col < 0 || col >= 2 * gt.Hv) continue;
          const float v = gdn::bf2f(gs[32 * (32 * i + r) + c]);
          if (col < gt.Hv) {
            gt.beta[static_cast<int64_t>(mm) * gt.Hv + col] = gdn::gate_beta(v);
          } else {
            const int h = col - gt.Hv;
            gt.g[static_cast<int64_t>(mm) * gt.Hv + h] =
                gdn::gate_g(v, gdn::load_param(gt.A_log, h, gt.param_f32), gdn::load_param(gt.dt_bias, h, gt.param_f32));
          }
        }
      }
    }
  }
}

// grid = 8 * ceil(tiles / 8); block = 256 (4 waves, 2 x 2 over the tile).
// Wave (wm, wn) owns rows BM / 2 wm .. and columns BN / 2 wn ..: MI x NJ
// accumulator tiles of 32 x 32 (MI = BM / 64, NJ = BN / 64).  kMinWG
// workgroups per CU bound the registers (1: 512 per lane, AGPRs included).
template <int BM, int BN, int kMinWG>
__global__ __launch_bounds__(kGemmThreads, kMinWG) void gemm_tn_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                                   const uint16_t* __restrict__ B, int64_t ldb,
                                                                   GemmOut out, int M,
                                                                   int N, int K, GemmGates gt) {
  constexpr int MI = BM / 64, NJ = BN / 64;
  constexpr int kStage = (BM + BN) * 128;  // bytes per stage: 64 KiB at 256 x 256
  constexpr int kPer = (BM + BN) / 32;     // 1 KiB blocks per wave per stage (= 2 (MI + NJ))
  constexpr int kAPer = BM / 32;           // of which A blocks (the first kAPer)
  constexpr int kReads = MI + NJ, kProds = MI * NJ;  // fragment reads, products per sub-step
  constexpr int kPair = kReads < kProds ? kReads : kProds;
  // two stages as two objects, so the compiler sees that products from one
  // do not read what the loads into the other write
  __shared__ __align__(16) uint8_t st0[kStage];
  __shared__ __align__(16) uint8_t st1[kStage];

  const int mb_n = (M + BM - 1) / BM, nb_n = (N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(mb_n) * nb_n;
  const int64_t L = gdn::xcd_remap(blockIdx.x, tiles);
  if (L < 0) return;
  // tile groups of kGroupM row blocks x all column blocks, row block fastest
  const int64_t per_group = static_cast<int64_t>(kGroupM) * nb_n;
  const int64_t grp = L / per_group, in_grp = L % per_group;
  const int gm = static_cast<int>(min<int64_t>(kGroupM, mb_n - grp * kGroupM));
  const int mb = static_cast<int>(grp * kGroupM + in_grp % gm);
  const int nb = static_cast<int>(in_grp / gm);
  const int m0 = mb * BM, n0 = nb * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lg = lane >> 5;

  // per-lane global byte offsets of the wave's kPer blocks (rows clamped:
  // rows past M (N) re-read the last row; their results are not stored)
  const __amdgpu_buffer_rsrc_t ra = rsrc_of(A), rb = rsrc_of(B);
  int goff[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = wave + 4 * i;
    const int gcol = 8 * ((lane & 7) ^ (((b & 1) << 2) | (lane >> 4)));
    if (i < kAPer) {
      goff[i] = static_cast<int>((min(m0 + 8 * b + (lane >> 3), M - 1) * lda + gcol) * 2);
    } else {
      goff[i] = static_cast<int>((min(n0 + 8 * (b - BM / 8) + (lane >> 3), N - 1) * ldb + gcol) * 2);
    }
  }
  const int nk = K / kBK;
  // the wave's blocks i0 .. i0 + n - 1 of step `step` (clamped to the last
  // step: the loads after the last step repeat it into the unused stage)
  auto issue = [&](uint8_t* st, int step, int i0, int n) {
    const int kbyte = min(step, nk - 1) * kBK * 2;
#pragma unroll
    for (int i = i0; i < i0 + n; ++i) dma16(i < kAPer ? ra : rb, st + (wave + 4 * i) * 1024, goff[i], kbyte);
  };

  f32x16_t acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = zero16();

  // Operand fragments of one 16-deep sub-step: MI of A, NJ of B (one 16-byte
  // LDS read each).  Fragments are read one sub-step ahead of their
  // products, so each read has a sub-step of products (512 cycles at 256 x
  // 256) to arrive.
  struct Frag {
    gdn::s16x8_t a[MI], b[NJ];
  };
  auto read_frag = [&](const uint8_t* st, int ks, Frag& f) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
      f.a[i] = *reinterpret_cast<const gdn::s16x8_t*>(st + sw_off((BM / 2) * wm + 32 * i + li, 2 * ks + lg));
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      f.b[j] = *reinterpret_cast<const gdn::s16x8_t*>(st + BM * 128 + sw_off((BN / 2) * wn + 32 * j + li, 2 * ks + lg));
  };
  // B as the first operand: the product is the tile of C^T, so each lane's
  // four consecutive accumulator registers are four consecutive columns of
  // one row of C (stored as one 8-byte piece)
  auto mfmas = [&](const Frag& f) {
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma_bf16(f.b[j], f.a[i], acc[i][j]);
  };
  // One sub-step's products with the next sub-step's reads between them.
  auto overlap = [&](const Frag& f, const uint8_t* st, int ks, Frag& nf) {
    read_frag(st, ks, nf);
    mfmas(f);
#pragma unroll
    for (int r = 0; r < kPair; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one product
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
    }
    if (kProds > kPair) __builtin_amdgcn_sched_group_barrier(0x008, kProds - kPair, 0);
    if (kReads > kPair) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPair, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // The same with half of the wave's loads of step `ld` into `dst` as well
  // (kPer / 2 = MI + NJ of them, one after each of the first products).  A
  // burst of loads stalls the wave (the address unit takes 1 KiB per 16
  // cycles, and four waves share it), so they are spread over the products.
  auto overlap_ld = [&](const Frag& f, const uint8_t* st, int ks, Frag& nf, uint8_t* dst, int ld, int i0) {
    read_frag(st, ks, nf);
    issue(dst, ld, i0, kPer / 2);
    mfmas(f);
#pragma unroll
    for (int r = 0; r < kPair; ++r) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one product
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
    }
    if (kProds > kPair) __builtin_amdgcn_sched_group_barrier(0x008, kProds - kPair, 0);
    if (kReads > kPair) {
      __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPair, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, kReads - kPair, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Step s (4 sub-steps) is multiplied from stage s % 2 while step s + 1 is
  // loaded into the other stage (during its first two sub-steps).  The barrier comes once the step's last
  // fragments are read (before their products): it waits for the wave's own
  // loads first, so after it the next stage is complete for every wave and
  // no wave reads the current stage any more (the loads of step s + 2 may
  // overwrite it).  The next step's first fragments are read behind the last
  // sub-step's products (no branch on the accumulators' path: a branch there
  // makes the compiler copy them and spill).
  Frag f0, f1;
  auto step = [&](uint8_t* cur, uint8_t* nxt, int s) {
    overlap_ld(f0, cur, 1, f1, nxt, s + 1, 0);
    overlap_ld(f1, cur, 2, f0, nxt, s + 1, kPer / 2);
    overlap(f0, cur, 3, f1);
    __syncthreads();
    overlap(f1, nxt, 0, f0);  // after the last step these reads go unused
  };
  issue(st0, 0, 0, kPer);
  __syncthreads();
  read_frag(st0, 0, f0);
  int s = 0;
  for (; s + 1 < nk; s += 2) {
    step(st0, st1, s);
    step(st1, st0, s + 1);
  }
  if (s < nk) step(st0, st1, s);  // the last step when nk is odd
  gemm_store<BM, BN>(acc, out, M, N, m0, n0, wave, lane, gt, nk % 2 ? st0 : st1);
}

// ---- small M (decode batches): a deeper load pipeline ----
// gemm_tn_kernel's two stages let a step's loads arrive during one step's
// products, which at 64-row tiles are four to eight products: every step then
// waits out the memory latency (its barrier drains every load).  Here the
// tile is 64 x BN and there are NS stages (3 or 4, separate LDS objects): the
// loads of step s + NS - 1 go out at the start of step s, and the barrier
// before step s waits only for the wave's loads of step s (vmcnt down to the
// NS - 2 later steps' loads) and for its own LDS reads (so every wave is done
// with the stage the next loads go into).  Same LDS layout, fragment reads,
// products in the same order and epilogue as gemm_tn_kernel: the results are
// the same bits.  Steps past the last one repeat its loads into the unused
// stages (every path issues the same loads), drained before the epilogue.
template <int BN, int NS>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_tn_deep_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                                    const uint16_t* __restrict__ B, int64_t ldb,
                                                                    GemmOut out, int M,
                                                                    int N, int K, GemmGates gt) {
  static_assert(NS == 3 || NS == 4, "three or four stages");
  constexpr int BM = 64, MI = 1, NJ = BN / 64;
  constexpr int kStage = (BM + BN) * 128;
  constexpr int kPer = (BM + BN) / 32;  // 1 KiB blocks per wave per stage
  constexpr int kAPer = BM / 32;
  // s_waitcnt: vmcnt = the NS - 2 later steps' loads (bits 3:0 and 15:14),
  // expcnt 7 (no wait), lgkmcnt 0
  constexpr int kVm = (NS - 2) * kPer;
  static_assert(kVm < 64, "vmcnt field");
  constexpr int kWait = (kVm & 15) | (7 << 4) | ((kVm >> 4) << 14);
  __shared__ __align__(16) uint8_t st0[kStage];
  __shared__ __align__(16) uint8_t st1[kStage];
  __shared__ __align__(16) uint8_t st2[kStage];
  __shared__ __align__(16) uint8_t st3[NS == 4 ? kStage : 16];

  const int mb_n = (M + BM - 1) / BM, nb_n = (N + BN - 1) / BN;
  const int64_t tiles = static_cast<int64_t>(mb_n) * nb_n;
  const int64_t L = gdn::xcd_remap(blockIdx.x, tiles);
  if (L < 0) return;
  const int64_t per_group = static_cast<int64_t>(kGroupM) * nb_n;
  const int64_t grp = L / per_group, in_grp = L % per_group;
  const int gm = static_cast<int>(min<int64_t>(kGroupM, mb_n - grp * kGroupM));
  const int mb = static_cast<int>(grp * kGroupM + in_grp % gm);
  const int nb = static_cast<int>(in_grp / gm);
  const int m0 = mb * BM, n0 = nb * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int li = lane & 31, lg = lane >> 5;

  const __amdgpu_buffer_rsrc_t ra = rsrc_of(A), rb = rsrc_of(B);
  int goff[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int b = wave + 4 * i;
    const int gcol = 8 * ((lane & 7) ^ (((b & 1) << 2) | (lane >> 4)));
    if (i < kAPer) {
      goff[i] = static_cast<int>((min(m0 + 8 * b + (lane >> 3), M - 1) * lda + gcol) * 2);
    } else {
      goff[i] = static_cast<int>((min(n0 + 8 * (b - BM / 8) + (lane >> 3), N - 1) * ldb + gcol) * 2);
    }
  }
  const int nk = K / kBK;
  auto issue = [&](uint8_t* st, int step) {
    const int kbyte = min(step, nk - 1) * kBK * 2;
#pragma unroll
    for (int i = 0; i < kPer; ++i) dma16(i < kAPer ? ra : rb, st + (wave + 4 * i) * 1024, goff[i], kbyte);
  };

  f32x16_t acc[MI][NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[0][j] = zero16();

  // one step from stage `cur`: the four sub-steps' fragments, then their products
  auto run = [&](const uint8_t* cur) {
    gdn::s16x8_t fa[4], fb[4][NJ];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      fa[ks] = *reinterpret_cast<const gdn::s16x8_t*>(cur + sw_off(32 * wm + li, 2 * ks + lg));
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        fb[ks][j] = *reinterpret_cast<const gdn::s16x8_t*>(cur + BM * 128 +
                                                           sw_off((BN / 2) * wn + 32 * j + li, 2 * ks + lg));
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[0][j] = mfma_bf16(fb[ks][j], fa[ks], acc[0][j]);
  };
  // step s from `cur`, the loads of step s + NS - 1 into `nxt` (the stage of
  // step s - 1, which every wave has finished reading at the barrier)
  auto one = [&](const uint8_t* cur, uint8_t* nxt, int step) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(kWait);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    issue(nxt, step + NS - 1);
    __builtin_amdgcn_sched_barrier(0);
    run(cur);
  };
  issue(st0, 0);
  issue(st1, 1);
  if constexpr (NS == 4) issue(st2, 2);
  // Two rounds of the stages per trip.  The compiler's load counting merges
  // its state at the loop head and then waits there for all but the newest
  // step's loads before the first reads (vmcnt(kPer)); within a trip the
  // barrier's own wait covers every read.
  for (int s = 0; s < nk; s += 2 * NS) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int s0 = s + r * NS;
      if constexpr (NS == 4) {
        if (s0 >= nk) break;
        one(st0, st3, s0);
        if (s0 + 1 >= nk) break;
        one(st1, st0, s0 + 1);
        if (s0 + 2 >= nk) break;
        one(st2, st1, s0 + 2);
        if (s0 + 3 >= nk) break;
        one(st3, st2, s0 + 3);
      } else {
        if (s0 >= nk) break;
        one(st0, st2, s0);
        if (s0 + 1 >= nk) break;
        one(st1, st0, s0 + 1);
        if (s0 + 2 >= nk) break;
        one(st2, st1, s0 + 2);
      }
    }
  }
  // the repeated loads land before a stage is reused as the gates' scratch
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  gemm_store<BM, BN>(acc, out, M, N, m0, n0, wave, lane, gt, st0);
}

}  // namespace

namespace {

// Tile choice and launch for C = A B^T into `out` (arguments checked by the
// entry points).
int gemm_launch(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, const GemmOut& out, int M, int N,
                int K, const GemmGates& gt, void* stream) {
  // Tile: 256 x 256 with one workgroup per CU, so a launch runs in
  // ceil(tiles / CUs) waves of tiles, each taking time in proportion to the
  // tile's rows.  192 x 256 is taken when its waves x rows is smaller (a
  // short last wave of 256-row tiles, e.g. 536 tiles = 2.09 waves -> 712 =
  // 2.78).  When 256 x 256 tiles would not fill half of the CUs (small M:
  // decode batches), 64 x 128 tiles, two or more workgroups per CU, spread
  // the work over the whole chip; 64 x 64 when even those would not.
  const int64_t nb256 = (N + 255) / 256;
  const int64_t t256 = ((M + 255) / 256) * nb256, t192 = ((M + 191) / 192) * nb256;
  const int64_t w256 = (t256 + kCUs - 1) / kCUs, w192 = (t192 + kCUs - 1) / kCUs;
  const int64_t t64x128 = ((M + 63) / 64) * ((N + 127) / 128);
  const int cfg = t256 >= kCUs / 2 ? (w192 * 192 < w256 * 256 ? 1 : 0) : t64x128 >= kCUs / 2 ? 2 : 3;
  const int64_t tiles = cfg == 3 ? ((M + 63) / 64) * ((N + 63) / 64) : cfg == 2 ? t64x128 : cfg == 1 ? t192 : t256;
  const int64_t grid = gdn::kNumXcd * ((tiles + gdn::kNumXcd - 1) / gdn::kNumXcd);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 g3(static_cast<unsigned>(grid)), b3(kGemmThreads);
  // The 64-row tiles take the deeper load pipeline when K has at least 16
  // steps (graph-replayed launches, 256 x 8224 x 2048: 21.1 -> 19.0 us; 256
  // x 2048 x 2048: 10.1 -> 9.3 us; 64 x 8224 x 2048: 17.2 -> 10.0 us); with
  // fewer its prologue and the repeated last loads cost more than it saves
  // (1000 x 2080 x 512: 6.5 -> 7.0 us).
  const bool deep = K / kBK >= 16;
  if (cfg == 3 && deep)
    gemm_tn_deep_kernel<64, 4><<<g3, b3, 0, st>>>(A, lda, B, ldb, out, M, N, K, gt);
  else if (cfg == 3)
    gemm_tn_kernel<64, 64, 2><<<g3, b3, 0, st>>>(A, lda, B, ldb, out, M, N, K, gt);
  else if (cfg == 2 && deep)
    gemm_tn_deep_kernel<128, 3><<<g3, b3, 0, st>>>(A, lda, B, ldb, out, M, N, K, gt);
  else if (cfg == 2)
    gemm_tn_kernel<64, 128, 2><<<g3, b3, 0, st>>>(A, lda, B, ldb, out, M, N, K, gt);
  else if (cfg == 1)
    gemm_tn_kernel<192, 256, 1><<<g3, b3, 0, st>>>(A, lda, B, ldb, out, M, N, K, gt);
  else
    gemm_tn_kernel<256, 256, 1><<<g3, b3, 0, st>>>(A, lda, B, ldb, out, M, N, K, gt);
  return gdn_launch_status();
}

// The checks both entry points share: K in steps of 64; 16-byte row pieces
// of A and B; 32-bit buffer offsets; the gate outputs' arguments.
int gemm_check(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, int M, int N, int K, float* g,
               uint16_t* beta, const void* A_log, const void* dt_bias, int gate_col, int Hv) {
  if (K % kBK || K == 0 || lda % 8 || ldb % 8 || lda < K || ldb < K || reinterpret_cast<uintptr_t>(A) % 16 ||
      reinterpret_cast<uintptr_t>(B) % 16 || static_cast<int64_t>(M) * lda * 2 >= (1LL << 31) ||
      static_cast<int64_t>(N) * ldb * 2 >= (1LL << 31))
    return GDN_ERR_INVALID_ARG;
  if (g && (!beta || !A_log || !dt_bias || Hv <= 0 || gate_col < 0 || gate_col + 2 * Hv > N)) return GDN_ERR_INVALID_ARG;
  return GDN_OK;
}

// One output part: rows of ld elements at c (16-byte stores when ld is a
// multiple of 8 and c 16-byte aligned, else element by element: c then only
// 2-byte aligned).
bool part_ok(const uint16_t* c, int64_t ld, int width) {
  return c && ld >= width && reinterpret_cast<uintptr_t>(c) % (ld % 8 ? 2 : 16) == 0;
}

}  // namespace

extern "C" int gdn_gemm_bf16(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, uint16_t* C,
                             int64_t ldc, int M, int N, int K, float* g, uint16_t* beta, const void* A_log,
                             const void* dt_bias, int param_is_fp32, int gate_col, int Hv, void* stream) {
  if (M < 0 || N < 0 || K < 0) return GDN_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return GDN_OK;
  if (!A || !B || !C) return GDN_ERR_INVALID_ARG;
  const int st = gemm_check(A, lda, B, ldb, M, N, K, g, beta, A_log, dt_bias, gate_col, Hv);
  if (st != GDN_OK) return st;
  if (!part_ok(C, ldc, N)) return GDN_ERR_INVALID_ARG;
  const int v = ldc % 8 == 0;
  const GemmOut out{{C, C, C, C}, {ldc, ldc, ldc, ldc}, {N, N, N, N}, {v, v, v, v}};
  const GemmGates gt{g, beta, A_log, dt_bias, param_is_fp32 ? 1 : 0, gate_col, Hv};
  return gemm_launch(A, lda, B, ldb, out, M, N, K, gt, stream);
}

extern "C" int gdn_gemm_bf16_cols(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb, int M, int N, int K,
                                  int n_parts, uint16_t* const* C, const int64_t* ldc, const int* col_end, float* g,
                                  uint16_t* beta, const void* A_log, const void* dt_bias, int param_is_fp32,
                                  int gate_col, int Hv, void* stream) {
  if (M < 0 || N < 0 || K < 0 || n_parts < 1 || n_parts > kMaxParts || !C || !ldc || !col_end)
    return GDN_ERR_INVALID_ARG;
  if (M == 0 || N == 0) return GDN_OK;
  if (!A || !B) return GDN_ERR_INVALID_ARG;
  const int st = gemm_check(A, lda, B, ldb, M, N, K, g, beta, A_log, dt_bias, gate_col, Hv);
  if (st != GDN_OK) return st;
  GemmOut out{};
  int beg = 0;
  for (int s = 0; s < kMaxParts; ++s) {
    const int e = s < n_parts ? col_end[s] : N;
    if (s < n_parts) {
      // increasing boundaries at multiples of 16, the last one at N
      if (e <= beg || (s + 1 < n_parts ? e % 16 != 0 || e >= N : e != N)) return GDN_ERR_INVALID_ARG;
      if (!part_ok(C[s], ldc[s], e - beg)) return GDN_ERR_INVALID_ARG;
      out.c[s] = C[s];
      out.ld[s] = ldc[s];
      out.vec[s] = ldc[s] % 8 == 0;
    } else {
      out.c[s] = out.c[n_parts - 1];
      out.ld[s] = out.ld[n_parts - 1];
      out.vec[s] = out.vec[n_parts - 1];
    }
    out.end[s] = e;
    beg = e;
  }
  const GemmGates gt{g, beta, A_log, dt_bias, param_is_fp32 ? 1 : 0, gate_col, Hv};
  return gemm_launch(A, lda, B, ldb, out, M, N, K, gt, stream);
}
