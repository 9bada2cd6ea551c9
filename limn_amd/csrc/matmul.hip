// Dense contraction on CDNA4 matrix cores: C[b, m, n] = sum_k A[b, m, k] * B[b, k, n] with bf16 or
// f16 operands, f32 accumulation, and an optional fused epilogue (relu) before the store.
//
// This is what a limn loop nest becomes when it is a dense contraction (a SUM over the last
// axis of a product of two buffers that share only the reduce and batch variables): the
// `A @ B` spelling of limn/tensor.py:486-496 lowers to exactly that nest (reference
// limn/cuda_emit.py:376-505 detects the same shape and emits a SIMT tile).
//
// Two kernels share the tiling. Output tiles are 256 x 256 (8 waves as 2 x 4, each owning
// 128 x 64 = 4 x 2 accumulators of v_mfma_f32_32x32x16) or 128 x 128 (4 waves as 2 x 2, each
// 64 x 64) when the larger tile would leave compute units idle. K advances BK = 64 per stage
// through two LDS buffers.
//
// matmul_dma (k a multiple of 64): operands go from memory straight into LDS by
// buffer_load ... lds (no VGPR staging, no LDS write instructions), the next stage's copy in
// flight while the current one is multiplied. Tiles are unpadded and XOR-swizzled, 16-byte
// chunk c of LDS row r at position c ^ f(r), so that the lane-linear DMA writes and the MFMA
// operand reads are both conflict-free: a k-contiguous operand's tile is [rows][64] with
// f(r) = (r >> 1) & 7 and each MFMA operand one ds_read_b128; an m- (or n-) contiguous operand's
// tile is [64][rows] with f(k) = (k & 3) << 2 and each MFMA operand two transposing
// ds_read_b64_tr_b16. Every wave's LDS reads for the next 16-deep k step are interleaved one per
// MFMA of the current step. The two buffers of each operand are separate __shared__ arrays and
// the loop is unrolled by two, so the compiler can see that a copy into the idle buffer never
// aliases a read of the current one (it would otherwise wait for the copy before every read).
//
// matmul_mfma (any k that is a multiple of 8): operands are loaded into registers through a
// buffer resource, the k tail past the end zeroed, and stored to padded LDS tiles ([rows][64 + 8]
// and [64][rows + 32]) with the same operand reads.
//
// Split k: a contraction whose output has too few tiles to give every CU a workgroup and whose k
// is long (a weight gradient sums over all batch rows) is cut into k slices; each workgroup
// computes one tile over one slice and writes float32 partials, and matmul_splits adds the
// slices per element in slice order, applies the epilogue and rounds, so the result does not
// depend on scheduling.
//
// Both kernels read operands through buffer resources: rows and k past an operand's end read as
// zeros, so the loops carry no bounds tests; only the epilogue checks m and n.

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

// The addends of one output cell: t is the contraction already rounded to T.
template <typename T>
__device__ __forceinline__ u16 bias_at(const MatmulAddends& add, int64_t col) {
  const int64_t i = col * add.bias_n;
  return add.bias_f32 ? T::pack(((const float*)add.bias)[i]) : ((const u16*)add.bias)[i];
}

template <typename T>
__device__ __forceinline__ u16 add_terms(u16 t, const MatmulAddends& add, int64_t bz, int64_t row, int64_t col) {
  float x = T::unpack(t);
  if (add.bias != nullptr) x = x + T::unpack(bias_at<T>(add, col));
  if (add.res != nullptr) x = T::unpack(add.res[bz * add.r_batch + row * add.r_m + col * add.r_n]) + x;
  return T::pack(x);
}

// The bias of 8 consecutive n (rounded to T when it is float32), and the residual of 8 consecutive
// n of one row: 16-byte loads where the terms are contiguous and aligned and the 8 cells lie before N (col is a multiple of 8), else
// element loads; cells past N read zeros (they are not stored).
template <typename T>
__device__ __forceinline__ u16x8 bias8(const MatmulAddends& add, int64_t col, int64_t N) {
  u16x8 v = zero8();
  if (add.bias == nullptr) return v;
  if ((add.vec & 1) && col + 7 < N) {
    if (!add.bias_f32) return *(const u16x8*)((const u16*)add.bias + col);
    const f32x4 lo = *(const f32x4*)((const float*)add.bias + col), hi = *(const f32x4*)((const float*)add.bias + col + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[e] = T::pack(lo[e]);
      v[e + 4] = T::pack(hi[e]);
    }
    return v;
  }
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = col + e < N ? bias_at<T>(add, col + e) : (u16)0;
  return v;
}
__device__ __forceinline__ u16x8 res8(const MatmulAddends& add, int64_t bz, int64_t row, int64_t col, int64_t N) {
  u16x8 v = zero8();
  if (add.res == nullptr) return v;
  const u16* r = add.res + bz * add.r_batch + row * add.r_m;
  if ((add.vec & 2) && col + 7 < N) return *(const u16x8*)(r + col);
#pragma unroll
  for (int e = 0; e < 8; e++) v[e] = col + e < N ? r[(col + e) * add.r_n] : (u16)0;
  return v;
}

// 8 rounded contraction cells (packed two to a word) with their terms added, rounded again: the
// two cells of a word unpacked from it and rounded back into one word together (pack2)
template <typename T>
__device__ __forceinline__ u32x4 add_terms8(u32x4 w, u16x8 bv, u16x8 rv, const MatmulAddends& add) {
  const u32x4 b = __builtin_bit_cast(u32x4, bv), r = __builtin_bit_cast(u32x4, rv);
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    float lo = T::unpack((u16)(w[e] & 0xFFFFu)), hi = T::unpack((u16)(w[e] >> 16));
    if (add.bias != nullptr) {
      lo = lo + T::unpack((u16)(b[e] & 0xFFFFu));
      hi = hi + T::unpack((u16)(b[e] >> 16));
    }
    if (add.res != nullptr) {
      lo = T::unpack((u16)(r[e] & 0xFFFFu)) + lo;
      hi = T::unpack((u16)(r[e] >> 16)) + hi;
    }
    out[e] = T::pack2(lo, hi);
  }
  return out;
}

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

  // the stage starting at k0; chunks at or past `depth` are zeroed (a k-contiguous row runs on
  // into the next row's elements there)
  __device__ __forceinline__ void load(int k0, int depth) {
#pragma unroll
    for (int s = 0; s < LOADS; s++) {
      const int c = threadIdx.x + s * MM_THREADS;
      const int lrow = c / PER_ROW, lcol = (c % PER_ROW) * 8;
      const int off = KCONTIG ? (row0 + lrow) * stride + k0 + lcol : (k0 + lrow) * stride + row0 + lcol;
      r[s] = __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, off * 2, 0, 0));
      if (KCONTIG && k0 + lcol >= depth) r[s] = zero8();
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

template <typename T, int BM, int BN, bool A_K, bool B_K, int EPI, bool PARTIAL>
__global__ __launch_bounds__(MM_THREADS, 1) void matmul_mfma(const u16* __restrict__ a, const u16* __restrict__ b,
                                                             u16* __restrict__ c, float* __restrict__ ws, MatmulShape s,
                                                             int64_t chunk, MatmulAddends add) {
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
  sa.load(kb, depth);
  sb.load(kb, depth);
  sa.store(As[0]);
  sb.store(Bs[0]);
  sa.load(kb + BK, depth);
  sb.load(kb + BK, depth);
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
    sa.load(kb + (st + 2) * BK, depth);
    sb.load(kb + (st + 2) * BK, depth);
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
          u16 t = T::pack(v);
          if (add.bias != nullptr || add.res != nullptr) t = add_terms<T>(t, add, bz, row, col);
          cbase[row * s.c_m + col * s.c_n] = t;
        }
      }
    }
}

// ---- matmul_dma ------------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void lds_void;

// the s_waitcnt immediate that waits for every outstanding vector memory operation (vmcnt 0) and
// leaves the other counters free
constexpr int WAIT_VMEM = 0x0F70;

// One operand's DMA copy into a swizzled LDS tile, and its MFMA operand reads.
template <int ROWS, bool KCONTIG, int WAVES>
struct DmaOperand {
  static constexpr int RB = KCONTIG ? BK * 2 : ROWS * 2;  // bytes per LDS row
  static constexpr int BYTES = (KCONTIG ? ROWS : BK) * RB;
  static constexpr int PASSES = BYTES / (1024 * WAVES);   // 1 KB DMA instructions per wave per stage
  static constexpr int RPI = 1024 / RB;                   // LDS rows one DMA instruction fills
  static constexpr int READS = KCONTIG ? 1 : 2;           // LDS reads per MFMA operand
  static_assert(PASSES * 1024 * WAVES == BYTES, "a stage is a whole number of DMA passes");
  static __device__ __forceinline__ int swizzle(int r) { return KCONTIG ? (r >> 1) & 7 : (r & 3) << 2; }

  const char* base;
  int64_t extent, step, first;  // bytes from base the operand spans; bytes per stage; first stage
  int voff[PASSES];

  __device__ __forceinline__ DmaOperand(const u16* b, int64_t rows, int64_t depth, int64_t stride, int64_t row0,
                                        int64_t k_lo, int wave, int lane) {
    base = (const char*)b;
    extent = 2 * (KCONTIG ? (rows - 1) * stride + depth : (depth - 1) * stride + rows);
    step = KCONTIG ? 2 * BK : 2 * BK * stride;
    first = k_lo / BK;
#pragma unroll
    for (int q = 0; q < PASSES; q++) {
      // lane `lane` of this wave's q-th instruction fills position `pos` of LDS row r
      const int r = (q * WAVES + wave) * RPI + lane / (RB / 16), pos = lane % (RB / 16);
      const int c = pos ^ swizzle(r);
      voff[q] = KCONTIG ? (int)(((row0 + r) * stride + c * 8) * 2) : (int)((r * stride + row0 + c * 8) * 2);
    }
  }

  // this wave's share of stage st into `tile`; a stage past the end reads zeros (or the next
  // slice's k) into the idle buffer, where nothing reads it
  __device__ __forceinline__ void copy(char* tile, int st, int wave) const {
    const int64_t off = (first + st) * step, left = extent - off;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)(base + off), (short)0, (int)(left > 0 ? left : 0), 0x00020000);
#pragma unroll
    for (int q = 0; q < PASSES; q++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)(tile + (q * WAVES + wave) * 1024), 16, voff[q], 0, 0, 0);
  }

  // per-lane read offsets for the T 32-row blocks a wave multiplies, starting at row `row0`: by
  // k step for a k-contiguous tile (the swizzle varies with k), by block otherwise
  template <int T>
  __device__ __forceinline__ void offsets(int row0, int lane, int* rd) const {
    if (KCONTIG) {
      const int r = lane & 31, h = lane >> 5;
#pragma unroll
      for (int kk = 0; kk < BK / 16; kk++) rd[kk] = (row0 + r) * RB + (((2 * kk + h) ^ swizzle(r)) & 7) * 16;
    } else {
      const int g = lane >> 4, i = lane & 15, k = 8 * (g >> 1) + (i >> 2);
#pragma unroll
      for (int t = 0; t < T; t++) {
        const int col = row0 + t * 32 + 16 * (g & 1) + 4 * (i & 3);
        rd[t] = k * RB + ((col >> 3) ^ swizzle(k)) * 16 + (col & 7) * 2;
      }
    }
  }

  // the MFMA operand of block t at k step kk: lane l gets X[row0 + 32 t + l % 32][16 kk + 8 (l / 32) + j]
  __device__ __forceinline__ u16x8 operand(const char* tile, const int* rd, int t, int kk) const {
    if (KCONTIG) return *(const u16x8*)(tile + rd[kk] + t * 32 * RB);
    // a transposing read gives lane i of each 16-lane group item j from the 8 bytes lane 4j + i/4
    // addresses, element i % 4: lane r addresses k row 16 kk + 8 (l / 32) + r / 4 (+ 4 for the
    // second read), columns row0 + 32 t + 16 ((l / 16) % 2) + 4 (r % 4)
    const char* p = tile + rd[t] + kk * 16 * RB;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p);
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + 4 * RB));
    return __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

template <int BM>
struct DmaTile {
  static constexpr int WAVES = BM == 256 ? 8 : 4;
  static constexpr int WN = WAVES / 2;  // waves along n; 2 along m
};

template <typename T, int BM, int BN, bool A_K, bool B_K, int EPI, bool PARTIAL>
__global__ __launch_bounds__(64 * DmaTile<BM>::WAVES, 2) void matmul_dma(const u16* __restrict__ a, const u16* __restrict__ b,
                                                                      u16* __restrict__ c, float* __restrict__ ws,
                                                                      MatmulShape s, int64_t chunk, int wide,
                                                                      MatmulAddends add) {
  constexpr int WAVES = DmaTile<BM>::WAVES, WN = DmaTile<BM>::WN;
  constexpr int WTM = BM / 2, WTN = BN / WN;  // one wave's output tile
  constexpr int TM = WTM / 32, TN = WTN / 32, KS = BK / 16;
  using DA = DmaOperand<BM, A_K, WAVES>;
  using DB = DmaOperand<BN, B_K, WAVES>;
  __shared__ __attribute__((aligned(1024))) char A0[DA::BYTES];
  __shared__ __attribute__((aligned(1024))) char A1[DA::BYTES];
  __shared__ __attribute__((aligned(1024))) char B0[DB::BYTES];
  __shared__ __attribute__((aligned(1024))) char B1[DB::BYTES];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n32 = lane & 31;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t tiles_n = (s.N + BN - 1) / BN, tiles_m = (s.M + BM - 1) / BM;
  const int64_t per_batch = tiles_m * tiles_n, per_slice = s.batch * per_batch;
  // workgroup b runs on XCD b % 8: renumber so each XCD takes a contiguous run of tiles, and walk
  // those in groups of 4 tile rows, so the rows and columns of operand an XCD's L2 holds are few
  int64_t id = blockIdx.x;
  if (gridDim.x % 8 == 0) id = (id % 8) * (gridDim.x / 8) + id / 8;
  const int64_t slice = id / per_slice;
  const int64_t bz = (id - slice * per_slice) / per_batch;
  const int64_t t = id - slice * per_slice - bz * per_batch;
  constexpr int64_t GROUP = 4;
  const int64_t group = t / (GROUP * tiles_n), first = group * GROUP;
  const int64_t rows = tiles_m - first < GROUP ? tiles_m - first : GROUP;
  const int64_t tm = first + (t - group * GROUP * tiles_n) % rows, tn = (t - group * GROUP * tiles_n) / rows;
  const int64_t m0 = tm * BM, n0 = tn * BN;
  const int64_t k_lo = slice * chunk, k_hi = k_lo + chunk < s.K ? k_lo + chunk : s.K;

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  const DA da(a + bz * s.a_batch, s.M, s.K, A_K ? s.a_m : s.a_k, m0, k_lo, wave, lane);
  const DB db(b + bz * s.b_batch, s.N, s.K, B_K ? s.b_n : s.b_k, n0, k_lo, wave, lane);
  int rda[A_K ? KS : TM], rdb[B_K ? KS : TN];
  da.template offsets<TM>(wm * WTM, lane, rda);
  db.template offsets<TN>(wn * WTN, lane, rdb);
  const int stages = (int)((k_hi - k_lo) / BK);

  u16x8 av[2][TM], bv[2][TN];
  auto read = [&](const char* at, const char* bt, int kk, u16x8* ao, u16x8* bo) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; i++) ao[i] = da.operand(at, rda, i, kk);
#pragma unroll
    for (int j = 0; j < TN; j++) bo[j] = db.operand(bt, rdb, j, kk);
  };
  // one stage on (at, bt) while stage st + 1 is copied into (an, bn)
  auto stage = [&](const char* at, const char* bt, char* an, char* bn, int st) __attribute__((always_inline)) {
    da.copy(an, st + 1, wave);
    db.copy(bn, st + 1, wave);
#pragma unroll
    for (int kk = 0; kk < KS; kk++) {
      const int p = kk & 1;
      if (kk + 1 < KS) read(at, bt, kk + 1, av[p ^ 1], bv[p ^ 1]);
      // the B operand goes first: each accumulator then holds C transposed, 4 consecutive n per lane
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = T::mfma32(bv[p][j], av[p][i], acc[i][j]);
    }
    // the copy first, then each MFMA of a k step paired with one LDS read for the next
    constexpr int RD = TM * DA::READS + TN * DB::READS, MF = TM * TN;
    __builtin_amdgcn_sched_group_barrier(0x020, DA::PASSES + DB::PASSES, 0);
#pragma unroll
    for (int kk = 0; kk < KS; kk++) {
      if (kk + 1 < KS) {
#pragma unroll
        for (int q = 0; q < (RD > MF ? RD : MF); q++) {
          if (q < MF) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          if (q < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      } else {
        __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);  // this wave's part of stage st + 1 has landed
    __syncthreads();                          // and every other wave's
    read(an, bn, 0, av[0], bv[0]);
  };

  da.copy(A0, 0, wave);
  db.copy(B0, 0, wave);
  __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
  __syncthreads();
  read(A0, B0, 0, av[0], bv[0]);
  for (int st = 0; st < stages; st += 2) {
    stage(A0, B0, A1, B1, st);
    if (st + 1 < stages) stage(A1, B1, A0, B0, st + 1);
  }

  // epilogue: lane holds C[m = wave row + 32 i + n32][n = wave column + 32 j + 8 q + 4 h + e],
  // e = 0..3 in items 4 q + e. Stored directly, each instruction would touch 32 rows with 16
  // bytes per row; instead the tile goes through the operand buffers, idle once every wave has
  // passed the barrier below. Each wave writes its 32-row blocks into a 16 KiB region of its own
  // (16-byte chunk c of staged row r at c ^ swz(r), so the writes are conflict-free), then reads
  // whole rows back, 16 bytes a lane, and each store instruction writes whole 128-byte (bf16) or
  // 256-byte (float32 partial) row segments of its wave's 64 columns. Measured on the MI355X,
  // identical results: (16384 x 2048, k = 512) 54.3 -> 42.4 us, (16384 x 512, k = 512) 16.6 ->
  // 13.4 us, 8192^3 1305 -> 1359 TFLOP/s; the direct stores had written at about 2.5 TB/s.
  __syncthreads();
  constexpr int ES = PARTIAL ? 4 : 2;     // bytes per stored element
  constexpr int RB = WTN * ES;            // bytes per staged row
  constexpr int CPR = RB / 16;            // 16-byte chunks per staged row
  constexpr int REGION = 16384;           // staging bytes per wave
  constexpr int IB = REGION / RB / 32 < TM ? REGION / RB / 32 : TM;  // 32-row blocks per pass
  constexpr int PER = WAVES / 4;          // wave regions per operand buffer
  constexpr int RPI = 64 / CPR;           // staged rows one read instruction covers
  static_assert(WTN == 64 && TM % IB == 0, "a wave's columns are one staged row");
  static_assert(DA::BYTES == REGION * PER && DB::BYTES == REGION * PER, "four buffers hold every wave's region");
  const int quarter = wave / PER;
  char* const region = (quarter == 0 ? A0 : quarter == 1 ? A1 : quarter == 2 ? B0 : B1) + (wave % PER) * REGION;
  auto swz = [](int r) __attribute__((always_inline)) { return CPR == 8 ? (r >> 1) & 7 : r & 15; };
#pragma unroll
  for (int p = 0; p < TM / IB; p++) {
#pragma unroll
    for (int ii = 0; ii < IB; ii++) {
      const int i = p * IB + ii, r = ii * 32 + n32;
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int q = 0; q < 4; q++) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            v[e] = acc[i][j][4 * q + e];
            if (!PARTIAL && EPI == MATMUL_EPILOGUE_RELU) v[e] = v[e] > 0.f ? v[e] : 0.f;
          }
          if (PARTIAL) {
            *(f32x4*)(region + r * RB + ((8 * j + 2 * q + h) ^ swz(r)) * 16) = f32x4{v[0], v[1], v[2], v[3]};
          } else {
            *(uint2*)(region + r * RB + ((4 * j + q) ^ swz(r)) * 16 + 8 * h) =
                make_uint2(T::pack2(v[0], v[1]), T::pack2(v[2], v[3]));
          }
        }
    }
    const int cc = lane % CPR;
    constexpr int ITS = IB * 32 / RPI;
    // the added terms first, every load in flight before the first store (as far as the compiler
    // knows the stores may alias them, so a load after a store would wait for it): the bias chunk
    // is the same for every row a lane stores, the residual one chunk per row
    const bool adds = !PARTIAL && (add.bias != nullptr || add.res != nullptr);
    u16x8 bv = zero8(), rv[ITS];
    if (adds) {
      const int64_t col = n0 + wn * WTN + cc * 8;
      bv = bias8<T>(add, col, s.N);
#pragma unroll
      for (int it = 0; it < ITS; it++) {
        const int64_t row = m0 + wm * WTM + p * IB * 32 + it * RPI + lane / CPR;
        rv[it] = row < s.M && col < s.N ? res8(add, bz, row, col, s.N) : zero8();
      }
    }
#pragma unroll
    for (int it = 0; it < ITS; it++) {
      const int r = it * RPI + lane / CPR;
      const u32x4 staged = *(const u32x4*)(region + r * RB + (cc ^ swz(r)) * 16);
      const int64_t row = m0 + wm * WTM + p * IB * 32 + r, col = n0 + wn * WTN + cc * (16 / ES);
      if (row >= s.M || col >= s.N) continue;
      if (PARTIAL) {
        const u32x4 w = staged;
        float* wp = ws + (slice * s.batch + bz) * s.M * s.N + row * s.N + col;
        if (wide && col + 3 < s.N) {
          *(u32x4*)wp = w;
        } else {
#pragma unroll
          for (int e = 0; e < 4; e++)
            if (col + e < s.N) wp[e] = __uint_as_float(w[e]);
        }
      } else {
        u16* o = c + bz * s.c_batch + row * s.c_m + col * s.c_n;
        const u32x4 w = adds ? add_terms8<T>(staged, bv, rv[it], add) : staged;
        if (wide == 2 && col + 7 < s.N) {
          *(u32x4*)o = w;
        } else if (wide && col + 7 < s.N) {
          *(uint2*)o = make_uint2(w[0], w[1]);
          *(uint2*)(o + 4) = make_uint2(w[2], w[3]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++)
            if (col + e < s.N) o[e * s.c_n] = (u16)(w[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
}

// Every instance the launcher below can pick, instantiated explicitly: hipcc (ROCm 7.2) leaves
// the host launch stubs of most implicitly instantiated instances of this kernel undefined,
// which makes the library fail to load.
#define LIMN_DMA_INSTANCE(T, BM, AK, BKC, EPI, P)                                                               \
  template __global__ void matmul_dma<T, BM, BM, AK, BKC, EPI, P>(const u16* __restrict__, const u16* __restrict__, \
                                                                  u16* __restrict__, float* __restrict__, MatmulShape, \
                                                                  int64_t, int, MatmulAddends);
#define LIMN_DMA_PARTIAL(T, BM, AK, BKC, EPI) LIMN_DMA_INSTANCE(T, BM, AK, BKC, EPI, false) LIMN_DMA_INSTANCE(T, BM, AK, BKC, EPI, true)
#define LIMN_DMA_EPILOGUE(T, BM, AK, BKC) \
  LIMN_DMA_PARTIAL(T, BM, AK, BKC, MATMUL_EPILOGUE_NONE) LIMN_DMA_PARTIAL(T, BM, AK, BKC, MATMUL_EPILOGUE_RELU)
#define LIMN_DMA_LAYOUT(T, BM)                                                                   \
  LIMN_DMA_EPILOGUE(T, BM, true, true) LIMN_DMA_EPILOGUE(T, BM, true, false) LIMN_DMA_EPILOGUE(T, BM, false, true) \
  LIMN_DMA_EPILOGUE(T, BM, false, false)
LIMN_DMA_LAYOUT(BF16, 256)
LIMN_DMA_LAYOUT(BF16, 128)
LIMN_DMA_LAYOUT(F16, 256)
LIMN_DMA_LAYOUT(F16, 128)
#undef LIMN_DMA_LAYOUT
#undef LIMN_DMA_EPILOGUE
#undef LIMN_DMA_PARTIAL
#undef LIMN_DMA_INSTANCE

// The slices of a split contraction, added per element in slice order, then the epilogue and the
// store at c's strides.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void matmul_splits(const float* __restrict__ ws, u16* __restrict__ c, MatmulShape s,
                                                     int64_t split, int quad, MatmulAddends add) {
  const bool adds = add.bias != nullptr || add.res != nullptr;
  const int64_t total = s.batch * s.M * s.N;
  if (quad) {
    // 4 consecutive n per thread (N % 4 == 0, output rows contiguous and 8-byte aligned): one
    // 16-byte load per slice, the row and column found once, one 8-byte store; each element's
    // slices are still added in slice order
    for (int64_t i = (blockIdx.x * (int64_t)256 + threadIdx.x) * 4; i < total; i += (int64_t)gridDim.x * 1024) {
      float4 v = *(const float4*)(ws + i);
      for (int64_t k = 1; k < split; k++) {
        const float4 w = *(const float4*)(ws + k * total + i);
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
      }
      if (EPI == MATMUL_EPILOGUE_RELU) {
        v.x = v.x > 0.f ? v.x : 0.f;
        v.y = v.y > 0.f ? v.y : 0.f;
        v.z = v.z > 0.f ? v.z : 0.f;
        v.w = v.w > 0.f ? v.w : 0.f;
      }
      const int64_t col = i % s.N, row = (i / s.N) % s.M, bz = i / (s.N * s.M);
      u16 t[4] = {T::pack(v.x), T::pack(v.y), T::pack(v.z), T::pack(v.w)};
      if (adds) {
#pragma unroll
        for (int e = 0; e < 4; e++) t[e] = add_terms<T>(t[e], add, bz, row, col + e);
      }
      const uint2 packed = {(unsigned)t[0] | ((unsigned)t[1] << 16), (unsigned)t[2] | ((unsigned)t[3] << 16)};
      *(uint2*)(c + bz * s.c_batch + row * s.c_m + col) = packed;
    }
    return;
  }
  for (int64_t i = blockIdx.x * (int64_t)256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    float v = ws[i];
    for (int64_t k = 1; k < split; k++) v += ws[k * total + i];
    if (EPI == MATMUL_EPILOGUE_RELU) v = v > 0.f ? v : 0.f;
    const int64_t col = i % s.N, row = (i / s.N) % s.M, bz = i / (s.N * s.M);
    const u16 t = T::pack(v);
    c[bz * s.c_batch + row * s.c_m + col * s.c_n] = adds ? add_terms<T>(t, add, bz, row, col) : t;
  }
}

template <typename T, int BM, int BN, bool A_K, bool B_K, int EPI>
int launch_tile(const void* a, const void* b, void* c, const MatmulShape& s, const MatmulPlan& plan,
                const MatmulAddends& add, void* ws, hipStream_t stream) {
  const int64_t blocks = plan.split * s.batch * ((s.M + BM - 1) / BM) * ((s.N + BN - 1) / BN);
  if (blocks > 0x7fffffff) return fail(LIMN_HIP_EUNSUPPORTED, "matmul: %lld workgroups exceed one launch", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(MM_THREADS);
  const bool tail = (s.K % BK) != 0 || (plan.chunk % BK) != 0;
  if (!tail) {
    // 16-byte stores (2) or 8-byte stores (1) of consecutive n when the output rows are
    // contiguous and that aligned; the float32 partials are dense, 16-byte aligned when N % 4 == 0
    const bool row8 = s.c_n == 1 && s.c_m % 4 == 0 && s.c_batch % 4 == 0 && (uintptr_t)c % 8 == 0;
    const bool row16 = s.c_n == 1 && s.c_m % 8 == 0 && s.c_batch % 8 == 0 && (uintptr_t)c % 16 == 0;
    const int wide = plan.split > 1 ? s.N % 4 == 0 : row16 ? 2 : row8 ? 1 : 0;
    const dim3 dma_block(64 * DmaTile<BM>::WAVES);
    if (plan.split == 1) {
      hipLaunchKernelGGL((matmul_dma<T, BM, BN, A_K, B_K, EPI, false>), grid, dma_block, 0, stream, (const u16*)a,
                         (const u16*)b, (u16*)c, (float*)nullptr, s, plan.chunk, wide, add);
      return check_hip(hipGetLastError(), "launching the matmul kernel");
    }
    hipLaunchKernelGGL((matmul_dma<T, BM, BN, A_K, B_K, EPI, true>), grid, dma_block, 0, stream, (const u16*)a,
                       (const u16*)b, (u16*)c, (float*)ws, s, plan.chunk, wide, add);
  } else if (plan.split == 1) {
    hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, false>), grid, block, 0, stream, (const u16*)a,
                       (const u16*)b, (u16*)c, (float*)nullptr, s, plan.chunk, add);
    return check_hip(hipGetLastError(), "launching the matmul kernel");
  } else {
    hipLaunchKernelGGL((matmul_mfma<T, BM, BN, A_K, B_K, EPI, true>), grid, block, 0, stream, (const u16*)a,
                       (const u16*)b, (u16*)c, (float*)ws, s, plan.chunk, add);
  }
  const int rc = check_hip(hipGetLastError(), "launching the split matmul kernel");
  if (rc != LIMN_HIP_OK) return rc;
  const int64_t total = s.batch * s.M * s.N;
  const bool quad = s.N % 4 == 0 && s.c_n == 1 && s.c_m % 4 == 0 && s.c_batch % 4 == 0 && (uintptr_t)c % 8 == 0;
  const int64_t per_thread = quad ? 4 : 1, threads = (total + per_thread - 1) / per_thread;
  const int64_t fold_blocks = (threads + 255) / 256 < 4096 ? (threads + 255) / 256 : 4096;
  hipLaunchKernelGGL((matmul_splits<T, EPI>), dim3((unsigned)fold_blocks), dim3(256), 0, stream, (const float*)ws,
                     (u16*)c, s, plan.split, (int)quad, add);
  return check_hip(hipGetLastError(), "launching the matmul slice fold");
}

template <typename T, bool A_K, bool B_K, int EPI>
int launch_layout(const void* a, const void* b, void* c, const MatmulShape& s, const MatmulPlan& plan,
                  const MatmulAddends& add, void* ws, hipStream_t stream) {
  if (plan.tile == 256) return launch_tile<T, 256, 256, A_K, B_K, EPI>(a, b, c, s, plan, add, ws, stream);
  return launch_tile<T, 128, 128, A_K, B_K, EPI>(a, b, c, s, plan, add, ws, stream);
}

template <typename T, int EPI>
int launch_type(const void* a, const void* b, void* c, const MatmulShape& s, const MatmulPlan& plan,
                const MatmulAddends& add, void* ws, hipStream_t stream) {
  const bool a_k = s.a_k == 1, b_k = s.b_k == 1;
  if (a_k && b_k) return launch_layout<T, true, true, EPI>(a, b, c, s, plan, add, ws, stream);
  if (a_k) return launch_layout<T, true, false, EPI>(a, b, c, s, plan, add, ws, stream);
  if (b_k) return launch_layout<T, false, true, EPI>(a, b, c, s, plan, add, ws, stream);
  return launch_layout<T, false, false, EPI>(a, b, c, s, plan, add, ws, stream);
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
// do; else k is split on 128 x 128 tiles, whose workgroups fit two to a CU: as many slices as
// fill every CU twice, each at least 2 * MIN_SLICE long (a multiple of BK); if slices that long
// cannot fill every CU once, the fewest slices at least MIN_SLICE long that do. Measured on the
// MI355X (the GPT weight gradients, K = 16384): (1536 x 512) 60.5 -> 38.9 us and (2048 x 512)
// 50.9 -> 45.9 us against 256 x 256 tiles cut into the fewest slices that fill every CU once,
// whose float32 partials moved twice the bytes; (512 x 512) keeps 16 slices of 1024 (32 slices
// of 512 took 26.0 us against 23.1).
MatmulPlan plan_matmul(const MatmulShape& s) {
  const int64_t t256 = s.batch * ((s.M + 255) / 256) * ((s.N + 255) / 256);
  const int64_t t128 = s.batch * ((s.M + 127) / 128) * ((s.N + 127) / 128);
  if (t256 >= FILL) return {256, 1, s.K};
  if (t128 >= FILL || s.K < 2 * MIN_SLICE) return {128, 1, s.K};
  int64_t split = 2 * FILL / t128, longest = s.K / (2 * MIN_SLICE);
  split = split < longest ? split : longest;
  if (split * t128 < FILL) {
    const int64_t most = s.K / MIN_SLICE;
    split = (FILL + t128 - 1) / t128;
    split = split < most ? split : most;
  }
  split = split > 1 ? split : 1;
  int64_t chunk = (s.K + split - 1) / split;
  chunk = (chunk + BK - 1) / BK * BK;
  return {128, (s.K + chunk - 1) / chunk, chunk};
}

int64_t matmul_workspace_bytes(const MatmulShape& s) {
  const MatmulPlan plan = plan_matmul(s);
  return plan.split > 1 ? plan.split * s.batch * s.M * s.N * (int64_t)sizeof(float) : 0;
}

int launch_matmul(const void* a, const void* b, void* c, int dtype, const MatmulShape& s, int epilogue,
                  const MatmulAddends& add, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  MatmulPlan plan = plan_matmul(s);
  if (plan.split > 1 && (workspace == nullptr || workspace_bytes < matmul_workspace_bytes(s)))
    plan = {plan.tile, 1, s.K};  // no room for the slices: the same contraction, unsplit
  const bool relu = epilogue == MATMUL_EPILOGUE_RELU;
  if (dtype == LIMN_HIP_BFLOAT16)
    return relu ? launch_type<BF16, MATMUL_EPILOGUE_RELU>(a, b, c, s, plan, add, workspace, stream)
                : launch_type<BF16, MATMUL_EPILOGUE_NONE>(a, b, c, s, plan, add, workspace, stream);
  return relu ? launch_type<F16, MATMUL_EPILOGUE_RELU>(a, b, c, s, plan, add, workspace, stream)
              : launch_type<F16, MATMUL_EPILOGUE_NONE>(a, b, c, s, plan, add, workspace, stream);
}

}  // namespace limn
