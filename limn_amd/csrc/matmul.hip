// Dense contraction on CDNA4 matrix cores: C[b, m, n] = sum_k A[b, m, k] * B[b, k, n] with bf16 or
// f16 operands, f32 accumulation, and an optional fused epilogue (relu) before the store.
//
// This is what a limn loop nest becomes when it is a dense contraction (a SUM over the last
// axis of a product of two buffers that share only the reduce and batch variables): the
// `A @ B` spelling of limn/tensor.py:486-496 lowers to exactly that nest (reference
// limn/cuda_emit.py:376-505 detects the same shape and emits a SIMT tile).
//
// Tiling: a 256-thread workgroup computes a BM x BN tile (256 x 256, or 128 x 128 when the
// larger tile would leave compute units idle); its 4 waves are 2 x 2, each owning
// (BM/2) x (BN/2) = TM x TN accumulators of v_mfma_f32_32x32x16 (32x32 outputs, 16-deep k per
// instruction), so per 16-deep step a wave reads TM + TN operands from LDS for TM * TN MFMAs.
// K advances BK = 64 per stage through a double-buffered LDS: the next stage's global loads are
// in registers while the current stage is multiplied.
//
// Split k: a contraction whose output has too few tiles to give every CU a workgroup and whose k
// is long (a weight gradient sums over all batch rows) is cut into k slices; each workgroup
// computes one tile over one slice and writes float32 partials, and matmul_splits adds the
// slices per element in slice order, applies the epilogue and rounds, so the result does not
// depend on scheduling.
//
// LDS holds both operands k-contiguous (A as [m][k], B as [n][k], rows padded by 8 elements
// so 16-byte reads across a 32-row operand are conflict-free), so each MFMA operand is one
// ds_read_b128. An operand that is k-contiguous in memory is staged with 16-byte row loads;
// one that is m- (or n-) contiguous is loaded 4 k-rows x 8 columns per thread and transposed
// in registers on the way into LDS, its k positions rotated per 16-row group so that those
// transposed writes spread over the banks.

#include "matmul.h"

namespace limn {
namespace {

constexpr int MM_THREADS = 256;
constexpr int BK = 64;
constexpr int LS = BK + 8;  // LDS row stride (elements) of both operand tiles

__device__ __forceinline__ u16x8 zero8() {
  u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  return z;
}

// k position of element k in LDS row `row` of an operand staged from row-contiguous memory:
// rotated by 8 per 16-row group (identity for k-contiguous staging). gfx950's LDS has 64
// four-byte banks and serves 16 lanes of a 16-byte read (32 lanes of an 8-byte write) per cycle.
// The row stride LS is 36 banks, so an operand read (16 consecutive rows, one rotation) starts
// in 16 distinct 4-bank groups; a staging write (rows 8 apart) would land every even and every
// odd row on one group, and the rotation by row >> 4 spreads them over all 16. Together with
// the lane-to-block map of OperandStage (k groups of opposite parity, 8 bytes apart, in the
// two 16-lane halves) the 32 lanes of a write fill all 64 banks.
template <bool KCONTIG>
__device__ __forceinline__ int kpos(int row, int k) {
  return KCONTIG ? k : ((k + 8 * ((row >> 4) & 7)) & (BK - 1));
}

// Block `blk` of a row-contiguous operand stage -> (8-row chunk rc, 4-deep k group kg): lanes
// 0-15 take 16 consecutive row chunks with an even k group, lanes 16-31 the same chunks with the
// next (odd) one; loads stay 256-byte coalesced per k row.
template <int ROWS>
__device__ __forceinline__ void stage_block(int blk, int& rc, int& kg) {
  constexpr int R16 = ROWS / 128;  // 16-chunk groups of rows
  rc = (blk & 15) | (((blk >> 5) % R16) << 4);
  kg = ((blk >> 4) & 1) | (((blk >> 5) / R16) << 1);
}

// One operand's stage: ROWS (m or n) x BK values, staged into an LDS tile [row][k].
//   KCONTIG: memory is k-contiguous: element (row, k) at base + row*stride + k.
//   else   : memory is row-contiguous: element (row, k) at base + k*stride + row.
template <int ROWS, bool KCONTIG>
struct OperandStage {
  static constexpr int LOADS = ROWS * BK / 8 / MM_THREADS;  // 16-byte loads per thread
  u16x8 r[LOADS];

  __device__ __forceinline__ void load(const u16* base, int64_t row0, int64_t rows, int64_t k0, int64_t depth,
                                       int64_t stride) {
    if (KCONTIG) {
#pragma unroll
      for (int s = 0; s < LOADS; s++) {
        const int c = threadIdx.x + s * MM_THREADS;
        const int row = c / (BK / 8), kc = c % (BK / 8);
        const int64_t gr = row0 + row, gk = k0 + kc * 8;
        r[s] = (gr < rows && gk < depth) ? *(const u16x8*)(base + gr * stride + gk) : zero8();
      }
    } else {
      // a block is 4 k-rows x 8 columns; column chunks vary fastest across lanes (coalesced)
#pragma unroll
      for (int s = 0; s < LOADS / 4; s++) {
        const int blk = threadIdx.x + s * MM_THREADS;
        int rc, kg;
        stage_block<ROWS>(blk, rc, kg);
        const int64_t gr = row0 + rc * 8;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int64_t gk = k0 + kg * 4 + e;
          r[4 * s + e] = (gr < rows && gk < depth) ? *(const u16x8*)(base + gk * stride + gr) : zero8();
        }
      }
    }
  }

  __device__ __forceinline__ void store(u16* lds) {
    if (KCONTIG) {
#pragma unroll
      for (int s = 0; s < LOADS; s++) {
        const int c = threadIdx.x + s * MM_THREADS;
        const int row = c / (BK / 8), kc = c % (BK / 8);
        *(u16x8*)(lds + row * LS + kc * 8) = r[s];
      }
    } else {
#pragma unroll
      for (int s = 0; s < LOADS / 4; s++) {
        const int blk = threadIdx.x + s * MM_THREADS;
        int rc, kg;
        stage_block<ROWS>(blk, rc, kg);
#pragma unroll
        for (int c = 0; c < 8; c++) {
          u16x4 t = {r[4 * s][c], r[4 * s + 1][c], r[4 * s + 2][c], r[4 * s + 3][c]};
          const int row = rc * 8 + c;
          *(u16x4*)(lds + row * LS + kpos<false>(row, kg * 4)) = t;
        }
      }
    }
  }
};

template <typename T, int BM, int BN, bool A_K, bool B_K, int EPI, bool PARTIAL>
__global__ __launch_bounds__(MM_THREADS, 1) void matmul_mfma(const u16* __restrict__ a, const u16* __restrict__ b,
                                                             u16* __restrict__ c, float* __restrict__ ws, MatmulShape s,
                                                             int64_t chunk) {
  constexpr int TM = BM / 64, TN = BN / 64;  // 32x32 accumulators per wave along m and n
  __shared__ __attribute__((aligned(16))) u16 As[2][BM * LS];
  __shared__ __attribute__((aligned(16))) u16 Bs[2][BN * LS];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n32 = lane & 31;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t tiles_n = (s.N + BN - 1) / BN, tiles_m = (s.M + BM - 1) / BM;
  const int64_t per_batch = tiles_m * tiles_n, per_slice = s.batch * per_batch;
  const int64_t slice = blockIdx.x / per_slice;  // 0 unless k is split
  const int64_t bz = (blockIdx.x - slice * per_slice) / per_batch;
  const int64_t t = blockIdx.x - slice * per_slice - bz * per_batch;
  const int64_t k_lo = slice * chunk, k_hi = k_lo + chunk < s.K ? k_lo + chunk : s.K;
  const int64_t tm = t / tiles_n, tn = t - tm * tiles_n;
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const u16* abase = a + bz * s.a_batch;
  const u16* bbase = b + bz * s.b_batch;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  OperandStage<BM, A_K> sa;
  OperandStage<BN, B_K> sb;
  const int64_t a_stride = A_K ? s.a_m : s.a_k;
  const int64_t b_stride = B_K ? s.b_n : s.b_k;
  const int stages = (int)((k_hi - k_lo + BK - 1) / BK);
  sa.load(abase, m0, s.M, k_lo, k_hi, a_stride);
  sb.load(bbase, n0, s.N, k_lo, k_hi, b_stride);
  sa.store(As[0]);
  sb.store(Bs[0]);
  __syncthreads();
  for (int st = 0; st < stages; st++) {
    const int cur = st & 1;
    if (st + 1 < stages) {
      sa.load(abase, m0, s.M, k_lo + (int64_t)(st + 1) * BK, k_hi, a_stride);
      sb.load(bbase, n0, s.N, k_lo + (int64_t)(st + 1) * BK, k_hi, b_stride);
    }
    const u16* at = As[cur];
    const u16* bt = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      u16x8 av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) {
        const int row = wm * (BM / 2) + i * 32 + n32;
        av[i] = *(const u16x8*)(at + row * LS + kpos<A_K>(row, kk * 16 + 8 * h));
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int row = wn * (BN / 2) + j * 32 + n32;
        bv[j] = *(const u16x8*)(bt + row * LS + kpos<B_K>(row, kk * 16 + 8 * h));
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = T::mfma32(av[i], bv[j], acc[i][j]);
    }
    if (st + 1 < stages) {
      sa.store(As[cur ^ 1]);
      sb.store(Bs[cur ^ 1]);
    }
    __syncthreads();
  }

  // epilogue: lane holds rows 8*(e/4) + 4h + e%4 of each 32x32 tile, column n32
  if (PARTIAL) {
    // this slice's float32 tile, element (slice, bz, row, col) of a dense [slice][batch][M][N]
    float* wbase = ws + (slice * s.batch + bz) * s.M * s.N;
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const int64_t col = n0 + wn * (BN / 2) + j * 32 + n32;
        if (col >= s.N) continue;
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
          if (row < s.M) wbase[row * s.N + col] = acc[i][j][e];
        }
      }
    return;
  }
  u16* cbase = c + bz * s.c_batch;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int64_t col = n0 + wn * (BN / 2) + j * 32 + n32;
      if (col >= s.N) continue;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int64_t row = m0 + wm * (BM / 2) + i * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
        if (row < s.M) {
          float v = acc[i][j][e];
          if (EPI == MATMUL_EPILOGUE_RELU) v = v > 0.f ? v : 0.f;
          cbase[row * s.c_m + col * s.c_n] = T::pack(v);
        }
      }
    }
}

// The slices of a split contraction, added per element in slice order, then the epilogue and the
// store at c's strides.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void matmul_splits(const float* __restrict__ ws, u16* __restrict__ c, MatmulShape s,
                                                     int64_t split) {
  const int64_t total = s.batch * s.M * s.N;
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    float v = ws[i];
    for (int64_t k = 1; k < split; k++) v += ws[k * total + i];
    if (EPI == MATMUL_EPILOGUE_RELU) v = v > 0.f ? v : 0.f;
    const int64_t col = i % s.N, row = (i / s.N) % s.M, bz = i / (s.N * s.M);
    c[bz * s.c_batch + row * s.c_m + col * s.c_n] = T::pack(v);
  }
}

template <typename T, int BM, int BN, bool A_K, bool B_K, int EPI>
int launch_tile(const void* a, const void* b, void* c, const MatmulShape& s, const MatmulPlan& plan, void* ws,
                hipStream_t stream) {
  const int64_t blocks = plan.split * s.batch * ((s.M + BM - 1) / BM) * ((s.N + BN - 1) / BN);
  if (blocks > 0x7fffffff) return fail(LIMN_HIP_EUNSUPPORTED, "matmul: %lld workgroups exceed one launch", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(MM_THREADS);
  if (plan.split == 1) {
    hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, false>), grid, block, 0, stream, (const u16*)a,
                       (const u16*)b, (u16*)c, (float*)nullptr, s, plan.chunk);
    return check_hip(hipGetLastError(), "launching the matmul kernel");
  }
  hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, true>), grid, block, 0, stream, (const u16*)a,
                     (const u16*)b, (u16*)c, (float*)ws, s, plan.chunk);
  const int rc = check_hip(hipGetLastError(), "launching the split matmul kernel");
  if (rc != LIMN_HIP_OK) return rc;
  const int64_t total = s.batch * s.M * s.N;
  const int64_t fold_blocks = (total + 255) / 256 < 4096 ? (total + 255) / 256 : 4096;
  hipLaunchKernelGGL((matmul_splits<T, EPI>), dim3((unsigned)fold_blocks), dim3(256), 0, stream, (const float*)ws,
                     (u16*)c, s, plan.split);
  return check_hip(hipGetLastError(), "launching the matmul slice fold");
}

template <typename T, bool A_K, bool B_K, int EPI>
int launch_layout(const void* a, const void* b, void* c, const MatmulShape& s, const MatmulPlan& plan, void* ws,
                  hipStream_t stream) {
  if (plan.tile == 256) return launch_tile<T, 256, 256, A_K, B_K, EPI>(a, b, c, s, plan, ws, stream);
  return launch_tile<T, 128, 128, A_K, B_K, EPI>(a, b, c, s, plan, ws, stream);
}

template <typename T, int EPI>
int launch_type(const void* a, const void* b, void* c, const MatmulShape& s, const MatmulPlan& plan, void* ws,
                hipStream_t stream) {
  const bool a_k = s.a_k == 1, b_k = s.b_k == 1;
  if (a_k && b_k) return launch_layout<T, true, true, EPI>(a, b, c, s, plan, ws, stream);
  if (a_k) return launch_layout<T, true, false, EPI>(a, b, c, s, plan, ws, stream);
  if (b_k) return launch_layout<T, false, true, EPI>(a, b, c, s, plan, ws, stream);
  return launch_layout<T, false, false, EPI>(a, b, c, s, plan, ws, stream);
}

constexpr int64_t FILL = 256;        // workgroups that give every CU one (one workgroup per CU fits)
constexpr int64_t MIN_SLICE = 512;   // shortest k slice worth its partial tile's round trip

}  // namespace

int matmul_layout_ok(const MatmulShape& s) {
  // one of the two strides of each operand must be 1, the other a multiple of 8 elements, so
  // every 16-byte load is aligned; the contiguous extent must be a multiple of 8 so that a
  // 16-byte chunk never straddles the end of a row
  const bool a_ok = (s.a_k == 1 && s.a_m % 8 == 0 && s.K % 8 == 0) || (s.a_m == 1 && s.a_k % 8 == 0 && s.M % 8 == 0);
  const bool b_ok = (s.b_k == 1 && s.b_n % 8 == 0 && s.K % 8 == 0) || (s.b_n == 1 && s.b_k % 8 == 0 && s.N % 8 == 0);
  const bool batch_ok = s.a_batch % 8 == 0 && s.b_batch % 8 == 0;
  return a_ok && b_ok && batch_ok;
}

// 256 x 256 tiles when they alone give every CU a workgroup; else 128 x 128 tiles when those
// do; else k is split, into the fewest slices (each at least MIN_SLICE long, a multiple of BK)
// that fill the machine, on 256 x 256 tiles if the slices can fill it that way, else 128 x 128.
MatmulPlan plan_matmul(const MatmulShape& s) {
  const int64_t t256 = s.batch * ((s.M + 255) / 256) * ((s.N + 255) / 256);
  const int64_t t128 = s.batch * ((s.M + 127) / 128) * ((s.N + 127) / 128);
  if (t256 >= FILL) return {256, 1, s.K};
  if (t128 >= FILL || s.K < 2 * MIN_SLICE) return {128, 1, s.K};
  const int64_t most = s.K / MIN_SLICE;
  auto cut = [&](int tile, int64_t tiles) -> MatmulPlan {
    int64_t split = (FILL + tiles - 1) / tiles;
    split = split < most ? split : most;
    int64_t chunk = (s.K + split - 1) / split;
    chunk = (chunk + BK - 1) / BK * BK;
    return {tile, (s.K + chunk - 1) / chunk, chunk};
  };
  const MatmulPlan big = cut(256, t256);
  if (big.split * t256 >= FILL) return big;
  return cut(128, t128);
}

int64_t matmul_workspace_bytes(const MatmulShape& s) {
  const MatmulPlan plan = plan_matmul(s);
  return plan.split > 1 ? plan.split * s.batch * s.M * s.N * (int64_t)sizeof(float) : 0;
}

int launch_matmul(const void* a, const void* b, void* c, int dtype, const MatmulShape& s, int epilogue, void* workspace,
                  int64_t workspace_bytes, hipStream_t stream) {
  MatmulPlan plan = plan_matmul(s);
  if (plan.split > 1 && (workspace == nullptr || workspace_bytes < matmul_workspace_bytes(s)))
    plan = {plan.tile, 1, s.K};  // no room for the slices: the same contraction, unsplit
  const bool relu = epilogue == MATMUL_EPILOGUE_RELU;
  if (dtype == LIMN_HIP_BFLOAT16)
    return relu ? launch_type<BF16, MATMUL_EPILOGUE_RELU>(a, b, c, s, plan, workspace, stream)
                : launch_type<BF16, MATMUL_EPILOGUE_NONE>(a, b, c, s, plan, workspace, stream);
  return relu ? launch_type<F16, MATMUL_EPILOGUE_RELU>(a, b, c, s, plan, workspace, stream)
              : launch_type<F16, MATMUL_EPILOGUE_NONE>(a, b, c, s, plan, workspace, stream);
}

}  // namespace limn
