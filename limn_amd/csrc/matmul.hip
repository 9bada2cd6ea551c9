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
// LDS holds each operand in its memory orientation, copied with 16-byte loads through a buffer
// resource (rows and k past the operand's end read as zeros, so the loop has no bounds tests). A
// k-contiguous operand's tile is [rows][64 + 8] and each MFMA operand is one ds_read_b128 of a
// row; an m- (or n-) contiguous operand's tile is [64][rows + 32] and each MFMA operand is two
// transposing ds_read_b64_tr_b16. The paddings make every LDS read and write conflict-free.

#include "matmul.h"

namespace limn {
namespace {

constexpr int MM_THREADS = 256;
constexpr int BK = 64;

__device__ __forceinline__ u16x8 zero8() {
  u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  return z;
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// One operand's LDS tile per stage, kept in its memory orientation:
//   k-contiguous operand -> [ROWS][BK + 8]: an MFMA operand is one ds_read_b128 of a row (the
//     row stride is 9 sixteen-byte groups, so the 16 rows a read serves per cycle hit 16 groups);
//   row-contiguous operand -> [BK][ROWS + 32]: an MFMA operand is two transposing
//     ds_read_b64_tr_b16 (a stride of 256 + 64 bytes puts the 4 k rows a 32-lane half reads into
//     4 different quarters of the 64 banks).
// Staging is plain 16-byte copies (8 consecutive lanes write 128 contiguous bytes): nothing is
// transposed in registers.
template <int ROWS, bool KCONTIG>
struct Operand {
  static constexpr int STRIDE = KCONTIG ? BK + 8 : ROWS + 32;
  static constexpr int ELEMS = STRIDE * (KCONTIG ? ROWS : BK);
  static constexpr int PER_ROW = KCONTIG ? BK / 8 : ROWS / 8;  // 16-byte chunks per LDS row
  static constexpr int LOADS = ROWS * BK / 8 / MM_THREADS;      // chunks per thread per stage
  __amdgpu_buffer_rsrc_t rsrc;
  int stride, row0;
  u16x8 r[LOADS];

  // base: the operand's batch slice; `rows` (m or n) and `depth` (k) bound the bytes the
  // resource covers, so rows or k beyond them read as zeros without a test
  __device__ __forceinline__ Operand(const u16* base, int64_t rows, int64_t depth, int64_t stride_, int64_t row0_) {
    stride = (int)stride_;
    row0 = (int)row0_;
    const int64_t extent = KCONTIG ? (rows - 1) * stride_ + depth : (depth - 1) * stride_ + rows;
    rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(extent * 2), 0x00020000);
  }

  // the stage starting at k0; chunks at or past `depth` are zeroed when TAIL (a k-contiguous row
  // runs on into the next row's elements there)
  template <bool TAIL>
  __device__ __forceinline__ void load(int k0, int depth) {
#pragma unroll
    for (int s = 0; s < LOADS; s++) {
      const int c = threadIdx.x + s * MM_THREADS;
      const int lrow = c / PER_ROW, lcol = (c % PER_ROW) * 8;
      const int off = KCONTIG ? (row0 + lrow) * stride + k0 + lcol : (k0 + lrow) * stride + row0 + lcol;
      r[s] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off * 2, 0, 0));
      if (TAIL && KCONTIG && k0 + lcol >= depth) r[s] = zero8();
    }
  }

  __device__ __forceinline__ void store(u16* lds) const {
#pragma unroll
    for (int s = 0; s < LOADS; s++) {
      const int c = threadIdx.x + s * MM_THREADS;
      *(u16x8*)(lds + (c / PER_ROW) * STRIDE + (c % PER_ROW) * 8) = r[s];
    }
  }

  // the MFMA operand of the 32 rows at `row` for the 16-deep k step kk: lane l gets
  // X[row + l % 32][16 kk + 8 (l / 32) + j], j = 0..7
  __device__ __forceinline__ u16x8 operand(const u16* lds, int row, int kk) const {
    const int lane = threadIdx.x & 63;
    if (KCONTIG) return *(const u16x8*)(lds + (row + (lane & 31)) * STRIDE + kk * 16 + 8 * (lane >> 5));
    // within each 16-lane group, lane i's item j' comes from the 8 bytes lane 4j' + i/4
    // addresses, element i % 4: lane r addresses k row 16kk + 8(l/32) + 4 inst + r/4, columns
    // row + 16((l/16) % 2) + 4(r % 4)
    const int g = lane >> 4, i = lane & 15;
    u16* p = (u16*)lds + (kk * 16 + 8 * (g >> 1) + (i >> 2)) * STRIDE + row + 16 * (g & 1) + 4 * (i & 3);
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p);
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 4 * STRIDE));
    return __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

template <typename T, int BM, int BN, bool A_K, bool B_K, int EPI, bool PARTIAL, bool TAIL>
__global__ __launch_bounds__(MM_THREADS, 1) void matmul_mfma(const u16* __restrict__ a, const u16* __restrict__ b,
                                                             u16* __restrict__ c, float* __restrict__ ws, MatmulShape s,
                                                             int64_t chunk) {
  constexpr int TM = BM / 64, TN = BN / 64;  // 32x32 accumulators per wave along m and n
  using OA = Operand<BM, A_K>;
  using OB = Operand<BN, B_K>;
  __shared__ __attribute__((aligned(16))) u16 As[2][OA::ELEMS];
  __shared__ __attribute__((aligned(16))) u16 Bs[2][OB::ELEMS];

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

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  OA sa(a + bz * s.a_batch, s.M, s.K, A_K ? s.a_m : s.a_k, m0);
  OB sb(b + bz * s.b_batch, s.N, s.K, B_K ? s.b_n : s.b_k, n0);
  const int stages = (int)((k_hi - k_lo + BK - 1) / BK);
  const int kb = (int)k_lo, depth = (int)k_hi;
  sa.template load<TAIL>(kb, depth);
  sb.template load<TAIL>(kb, depth);
  sa.store(As[0]);
  sb.store(Bs[0]);
  sa.template load<TAIL>(kb + BK, depth);
  sb.template load<TAIL>(kb + BK, depth);
  __syncthreads();
  // one basic block per stage: the next stage's stores and the one after's loads are
  // unconditional (past the last stage they fill the idle buffer, or read zeros), so the compiler
  // can interleave them with the MFMAs
  for (int st = 0; st < stages; st++) {
    const int cur = st & 1;
    const u16* at = As[cur];
    const u16* bt = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK / 16; kk++) {
      u16x8 av[TM], bv[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) av[i] = sa.operand(at, wm * (BM / 2) + i * 32, kk);
#pragma unroll
      for (int j = 0; j < TN; j++) bv[j] = sb.operand(bt, wn * (BN / 2) + j * 32, kk);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = T::mfma32(av[i], bv[j], acc[i][j]);
    }
    sa.store(As[cur ^ 1]);
    sb.store(Bs[cur ^ 1]);
    sa.template load<TAIL>(kb + (st + 2) * BK, depth);
    sb.template load<TAIL>(kb + (st + 2) * BK, depth);
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
  const bool tail = (s.K % BK) != 0 || (plan.chunk % BK) != 0;
  if (plan.split == 1) {
    if (tail)
      hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, false, true>), grid, block, 0, stream, (const u16*)a,
                         (const u16*)b, (u16*)c, (float*)nullptr, s, plan.chunk);
    else
      hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, false, false>), grid, block, 0, stream, (const u16*)a,
                         (const u16*)b, (u16*)c, (float*)nullptr, s, plan.chunk);
    return check_hip(hipGetLastError(), "launching the matmul kernel");
  }
  if (tail)
    hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, true, true>), grid, block, 0, stream, (const u16*)a,
                       (const u16*)b, (u16*)c, (float*)ws, s, plan.chunk);
  else
    hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, true, false>), grid, block, 0, stream, (const u16*)a,
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
  // the kernel addresses each operand's batch slice through a buffer resource with 32-bit byte
  // offsets; a tile overhanging the last row or the last stage by up to 256 rows or 3 stages
  // must still be addressable
  auto reach = [](int64_t rows, int64_t depth, int64_t row_stride, int64_t k_stride) {
    return ((rows + 256) * row_stride + (depth + 3 * BK) * k_stride + 256) * 2;
  };
  const bool reach_ok = reach(s.M, s.K, s.a_m, s.a_k) < INT32_MAX && reach(s.N, s.K, s.b_n, s.b_k) < INT32_MAX;
  return a_ok && b_ok && batch_ok && reach_ok;
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
