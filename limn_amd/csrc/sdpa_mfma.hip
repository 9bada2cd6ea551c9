// Flash attention on CDNA4 matrix cores: bf16/f16 storage, f32 accumulation and softmax
// statistics, head dim D in {64, 128} (hd == hd_v). Forward, dQ pass and dK/dV pass, the
// three CUSTOM kernels limn's attention seam asks for (reference limn/tensor.py:509-575,
// 679-714), each deterministic: every total is accumulated inside one wave in a fixed order.
//
// Work decomposition (all three kernels):
//   a workgroup is 4 waves and owns BLOCK_ROWS = 128 *resident* rows (queries for the forward
//   and dQ pass, keys for the dK/dV pass), 32 per wave; the other side *streams* past in tiles
//   of TILE = 64 rows staged through LDS, the next tile's global loads in flight while the
//   current one is computed.
//
// Orientation. Every product is v_mfma_f32_32x32x16_{bf16,f16} with the resident rows on the
// N side, so each lane owns one resident row (n = lane % 32) and its score column is spread
// over the lane's 16 accumulator items (two lanes, lane and lane ^ 32, share a row):
//   forward:  S^T = K Q^T      then  O^T  += V^T P^T
//   dQ pass:  S^T = K Q^T, dP^T = V dO^T,  dQ^T += K^T dS^T
//   dKV pass: S = Q K^T, dP = dO V^T,      dV^T += dO^T P,  dK^T += Q^T dS
// A row's softmax statistics are then lane-local (the forward's running max needs one
// exchange with lane ^ 32 per tile), and a probability tile converted to bf16 *is* the
// B operand of the next product without moving between lanes: the accumulator items 8c..8c+7
// of a lane cover 8 of the 16 streamed rows of k-chunk c. The A operand of that product
// reads the streamed operand transposed; it is staged into LDS transposed with its rows
// permuted (tpos) so that those same 8 rows sit in one 16-byte LDS word.
//
// 32x32 accumulator layout (CDNA3/CDNA4 matrix cores): lane l, item i holds
// row 8*(i/4) + 4*(l/32) + i%4, column l%32.

#include "sdpa.h"

namespace limn {
namespace {

constexpr int WAVES = 4;
constexpr int THREADS = 64 * WAVES;
constexpr int BLOCK_ROWS = 32 * WAVES;
constexpr int TILE = 64;
constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// Position of streamed row r (0..TILE-1) in a transposed LDS tile: within each 32-row
// sub-tile the 4-row groups g = 4c + 2q + h are reordered to 4c + 2h + q, so the 8 rows
// {16c + 8q + 4h + e} that lane half h feeds to k-chunk c are contiguous at 16c + 8h.
__device__ __forceinline__ int tpos(int r) {
  const int g = (r >> 2) & 7;
  const int gp = (g & 4) | ((g & 1) << 1) | ((g >> 1) & 1);
  return (r & ~31) | (gp << 2) | (r & 3);
}

// A transposed tile's row `d` stores its TILE positions rotated by 8 * ((d >> 3) & 7): the
// staging writes 8 rows apart then land in 8 different 16-byte bank groups, while an MFMA
// operand read (8 consecutive positions starting at a multiple of 8, one row per lane)
// stays one contiguous 16-byte word.
__device__ __forceinline__ int trot(int d, int pos) { return (pos + 8 * ((d >> 3) & 7)) & (TILE - 1); }

__device__ __forceinline__ u16x8 zero8() {
  u16x8 z = {0, 0, 0, 0, 0, 0, 0, 0};
  return z;
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; i++) z[i] = 0.f;
  return z;
}

// Global -> registers -> LDS staging of one or two TILE x D row-major tiles. Each participating
// thread carries a 4-row x 8-column block, so it can write its rows (16 B per row) into a
// row-major LDS tile and its columns (8 B per column, 4 rows) into a transposed one.
template <int D>
struct Stage {
  static constexpr int COLS = D / 8;           // 16-byte column chunks per row
  static constexpr int PER_TILE = COLS * (TILE / 4);
  static constexpr int SLOTS = (2 * PER_TILE + THREADS - 1) / THREADS;  // both tiles
  u16x8 r[SLOTS][4];

  // Load tile `which` (0 or 1) of a pair: rows [row0, row0 + TILE) of base (rows x D), zero
  // past `rows`.
  __device__ __forceinline__ void load(const u16* base0, const u16* base1, int64_t row0, int64_t rows) {
#pragma unroll
    for (int s = 0; s < SLOTS; s++) {
      const int idx = threadIdx.x + s * THREADS;
      if (idx < 2 * PER_TILE) {
        const int which = idx / PER_TILE, w = idx - which * PER_TILE;
        const int col = w % COLS, grp = w / COLS;
        const u16* base = which ? base1 : base0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int64_t row = row0 + grp * 4 + e;
          r[s][e] = row < rows ? *(const u16x8*)(base + row * D + col * 8) : zero8();
        }
      }
    }
  }

  // rows0/cols0 receive tile 0, rows1/cols1 tile 1; a null destination is skipped.
  __device__ __forceinline__ void store(u16* rows0, u16* cols0, u16* rows1, u16* cols1) {
    constexpr int RS = D + 8, CS = TILE + 8;
#pragma unroll
    for (int s = 0; s < SLOTS; s++) {
      const int idx = threadIdx.x + s * THREADS;
      if (idx < 2 * PER_TILE) {
        const int which = idx / PER_TILE, w = idx - which * PER_TILE;
        const int col = w % COLS, grp = w / COLS;
        u16* rows = which ? rows1 : rows0;
        u16* cols = which ? cols1 : cols0;
        if (rows != nullptr) {
#pragma unroll
          for (int e = 0; e < 4; e++) *(u16x8*)(rows + (grp * 4 + e) * RS + col * 8) = r[s][e];
        }
        if (cols != nullptr) {
          const int p = tpos(grp * 4);
#pragma unroll
          for (int c = 0; c < 8; c++) {
            u16x4 t = {r[s][0][c], r[s][1][c], r[s][2][c], r[s][3][c]};
            const int d = col * 8 + c;
            *(u16x4*)(cols + d * CS + trot(d, p)) = t;
          }
        }
      }
    }
  }
};

// acc (32 rows x 32 cols per tile, row = dim d, col = resident row n) -> global (rows, D),
// scaled by `mul`, for the lane's resident row `row` if it is < rows.
template <typename T, int D>
__device__ __forceinline__ void store_transposed(u16* base, const f32x16* acc, int64_t row, int64_t rows, float mul) {
  if (row >= rows) return;
  const int h = (threadIdx.x >> 5) & 1;
#pragma unroll
  for (int dt = 0; dt < D / 32; dt++) {
#pragma unroll
    for (int g = 0; g < 4; g++) {
      u16x4 o = {T::pack(acc[dt][4 * g] * mul), T::pack(acc[dt][4 * g + 1] * mul), T::pack(acc[dt][4 * g + 2] * mul),
                 T::pack(acc[dt][4 * g + 3] * mul)};
      *(u16x4*)(base + row * D + dt * 32 + 8 * g + 4 * h) = o;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Forward.
template <typename T, int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 2) void sdpa_fwd_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                            const u16* __restrict__ v, const u16* __restrict__ mask,
                                                            u16* __restrict__ out, float* __restrict__ lse, int64_t batch,
                                                            int64_t t_q, int64_t t_k, float scale) {
  constexpr int RS = D + 8, CS = TILE + 8;
  __shared__ __attribute__((aligned(16))) u16 Ks[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Vt[D * CS];
  __shared__ float Mk[TILE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + BLOCK_ROWS - 1) / BLOCK_ROWS;
  const int64_t b = blockIdx.x % batch;
  const int64_t qb = nqb - 1 - blockIdx.x / batch;  // causal: the longest rows go first
  const int64_t q0 = qb * BLOCK_ROWS, wq0 = q0 + wave * 32, row = wq0 + n;
  const u16* qbase = q + b * t_q * D;
  const u16* kbase = k + b * t_k * D;
  const u16* vbase = v + b * t_k * D;
  const float c2 = scale * LOG2E;

  u16x8 qf[D / 16];
#pragma unroll
  for (int ds = 0; ds < D / 16; ds++) qf[ds] = row < t_q ? *(const u16x8*)(qbase + row * D + ds * 16 + 8 * h) : zero8();

  f32x16 acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; dt++) acc[dt] = zero16();
  float m = neg_inf(), l = 0.f;

  const int64_t kend = CAUSAL ? (q0 + BLOCK_ROWS < t_k ? q0 + BLOCK_ROWS : t_k) : t_k;
  const int ntiles = (int)((kend + TILE - 1) / TILE);
  Stage<D> st;
  st.load(kbase, vbase, 0, t_k);
  for (int it = 0; it < ntiles; it++) {
    const int64_t k0 = (int64_t)it * TILE;
    if (it > 0) __syncthreads();
    st.store(Ks, nullptr, nullptr, Vt);
    if (MASK && threadIdx.x < TILE) {
      const int64_t key = k0 + threadIdx.x;
      Mk[threadIdx.x] = key < t_k ? T::unpack(mask[b * t_k + key]) : 0.f;
    }
    __syncthreads();
    if (it + 1 < ntiles) st.load(kbase, vbase, k0 + TILE, t_k);
    if (CAUSAL && k0 > wq0 + 31) continue;  // every key of this tile is right of this wave's rows

    f32x16 s[2];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      s[sub] = zero16();
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++) {
        const u16x8 a = *(const u16x8*)(Ks + (sub * 32 + n) * RS + ds * 16 + 8 * h);
        s[sub] = T::mfma32(a, qf[ds], s[sub]);
      }
    }
    const bool edge = (k0 + TILE > t_k) || MASK || (CAUSAL && k0 + TILE - 1 > wq0);
    if (edge) {
#pragma unroll
      for (int sub = 0; sub < 2; sub++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int r = sub * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          const int64_t key = k0 + r;
          const bool hide = key >= t_k || (CAUSAL && key > row) || (MASK && Mk[r] == 0.f);
          if (hide) s[sub][i] = neg_inf();
        }
    }
    float mx = neg_inf();
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int i = 0; i < 16; i++) mx = fmaxf(mx, s[sub][i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mnew = fmaxf(m, mx);
    const float base = mnew == neg_inf() ? 0.f : mnew * c2;
    const float alpha = fast_exp2(m * c2 - base);
    float rs = 0.f;
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float p = fast_exp2(fmaf(s[sub][i], c2, -base));
        s[sub][i] = p;
        rs += p;
      }
    l = fmaf(l, alpha, rs);
    m = mnew;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) acc[dt] *= alpha;
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 pb;
#pragma unroll
        for (int j = 0; j < 8; j++) pb[j] = T::pack(s[sub][8 * c + j]);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          const int d = dt * 32 + n;
          const u16x8 a = *(const u16x8*)(Vt + d * CS + trot(d, sub * 32 + 16 * c + 8 * h));
          acc[dt] = T::mfma32(a, pb, acc[dt]);
        }
      }
  }
  const float total = l + __shfl_xor(l, 32);
  store_transposed<T, D>(out + b * t_q * D, acc, row, t_q, 1.f / total);
  if (h == 0 && row < t_q) lse[b * t_q + row] = m * scale + logf(total);
}

// ---------------------------------------------------------------------------------------------
// dQ pass: resident query rows, keys streaming.
template <typename T, int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 1) void sdpa_bwd_q_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                              const u16* __restrict__ v, const u16* __restrict__ dout,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ delta,
                                                              const u16* __restrict__ mask, u16* __restrict__ dq,
                                                              int64_t batch, int64_t t_q, int64_t t_k, float scale) {
  constexpr int RS = D + 8, CS = TILE + 8;
  __shared__ __attribute__((aligned(16))) u16 Ks[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Vs[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Kt[D * CS];
  __shared__ float Mk[TILE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + BLOCK_ROWS - 1) / BLOCK_ROWS;
  const int64_t b = blockIdx.x % batch;
  const int64_t qb = nqb - 1 - blockIdx.x / batch;
  const int64_t q0 = qb * BLOCK_ROWS, wq0 = q0 + wave * 32, row = wq0 + n;
  const u16* qbase = q + b * t_q * D;
  const u16* obase = dout + b * t_q * D;
  const u16* kbase = k + b * t_k * D;
  const u16* vbase = v + b * t_k * D;
  const float c2 = scale * LOG2E;

  u16x8 qf[D / 16], of[D / 16];
#pragma unroll
  for (int ds = 0; ds < D / 16; ds++) {
    qf[ds] = row < t_q ? *(const u16x8*)(qbase + row * D + ds * 16 + 8 * h) : zero8();
    of[ds] = row < t_q ? *(const u16x8*)(obase + row * D + ds * 16 + 8 * h) : zero8();
  }
  const float L2 = row < t_q ? lse[b * t_q + row] * LOG2E : 0.f;
  const float Dr = row < t_q ? delta[b * t_q + row] : 0.f;

  f32x16 acc[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; dt++) acc[dt] = zero16();

  const int64_t kend = CAUSAL ? (q0 + BLOCK_ROWS < t_k ? q0 + BLOCK_ROWS : t_k) : t_k;
  const int ntiles = (int)((kend + TILE - 1) / TILE);
  Stage<D> st;
  st.load(kbase, vbase, 0, t_k);
  for (int it = 0; it < ntiles; it++) {
    const int64_t k0 = (int64_t)it * TILE;
    if (it > 0) __syncthreads();
    st.store(Ks, Kt, Vs, nullptr);
    if (MASK && threadIdx.x < TILE) {
      const int64_t key = k0 + threadIdx.x;
      Mk[threadIdx.x] = key < t_k ? T::unpack(mask[b * t_k + key]) : 0.f;
    }
    __syncthreads();
    if (it + 1 < ntiles) st.load(kbase, vbase, k0 + TILE, t_k);
    if (CAUSAL && k0 > wq0 + 31) continue;

    f32x16 s[2], dp[2];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      s[sub] = zero16();
      dp[sub] = zero16();
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++) {
        const u16x8 a = *(const u16x8*)(Ks + (sub * 32 + n) * RS + ds * 16 + 8 * h);
        s[sub] = T::mfma32(a, qf[ds], s[sub]);
        const u16x8 e = *(const u16x8*)(Vs + (sub * 32 + n) * RS + ds * 16 + 8 * h);
        dp[sub] = T::mfma32(e, of[ds], dp[sub]);
      }
    }
    const bool edge = (k0 + TILE > t_k) || MASK || (CAUSAL && k0 + TILE - 1 > wq0);
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        float p = fast_exp2(fmaf(s[sub][i], c2, -L2));
        if (edge) {
          const int r = sub * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          const int64_t key = k0 + r;
          const bool hide = key >= t_k || (CAUSAL && key > row) || (MASK && Mk[r] == 0.f);
          if (hide) p = 0.f;
        }
        s[sub][i] = p * (dp[sub][i] - Dr) * scale;
      }
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 g;
#pragma unroll
        for (int j = 0; j < 8; j++) g[j] = T::pack(s[sub][8 * c + j]);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          const int d = dt * 32 + n;
          const u16x8 a = *(const u16x8*)(Kt + d * CS + trot(d, sub * 32 + 16 * c + 8 * h));
          acc[dt] = T::mfma32(a, g, acc[dt]);
        }
      }
  }
  store_transposed<T, D>(dq + b * t_q * D, acc, row, t_q, 1.f);
}

// ---------------------------------------------------------------------------------------------
// dK/dV pass: resident key rows, queries streaming.
template <typename T, int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 1) void sdpa_bwd_kv_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                               const u16* __restrict__ v, const u16* __restrict__ dout,
                                                               const float* __restrict__ lse,
                                                               const float* __restrict__ delta,
                                                               const u16* __restrict__ mask, u16* __restrict__ dk,
                                                               u16* __restrict__ dv, int64_t batch, int64_t t_q,
                                                               int64_t t_k, float scale) {
  constexpr int RS = D + 8, CS = TILE + 8;
  __shared__ __attribute__((aligned(16))) u16 Qs[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Os[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Qt[D * CS];
  __shared__ __attribute__((aligned(16))) u16 Ot[D * CS];
  __shared__ __attribute__((aligned(16))) float Ls[TILE];
  __shared__ __attribute__((aligned(16))) float Ds[TILE];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, h = lane >> 5, n = lane & 31;
  const int64_t b = blockIdx.x % batch;
  const int64_t kb = blockIdx.x / batch;  // causal: the first keys are seen by the most queries
  const int64_t k0 = kb * BLOCK_ROWS, wk0 = k0 + wave * 32, key = wk0 + n;
  const u16* qbase = q + b * t_q * D;
  const u16* obase = dout + b * t_q * D;
  const u16* kbase = k + b * t_k * D;
  const u16* vbase = v + b * t_k * D;
  const float c2 = scale * LOG2E;

  u16x8 kf[D / 16], vf[D / 16];
#pragma unroll
  for (int ds = 0; ds < D / 16; ds++) {
    kf[ds] = key < t_k ? *(const u16x8*)(kbase + key * D + ds * 16 + 8 * h) : zero8();
    vf[ds] = key < t_k ? *(const u16x8*)(vbase + key * D + ds * 16 + 8 * h) : zero8();
  }
  const bool live = key < t_k && (!MASK || T::unpack(mask[b * t_k + key]) != 0.f);

  f32x16 gk[D / 32], gv[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; dt++) {
    gk[dt] = zero16();
    gv[dt] = zero16();
  }

  const int64_t qstart = CAUSAL ? k0 : 0;  // a causal key is seen by queries at or after it
  const int ntiles = qstart < t_q ? (int)((t_q - qstart + TILE - 1) / TILE) : 0;
  Stage<D> st;
  if (ntiles > 0) st.load(qbase, obase, qstart, t_q);
  for (int it = 0; it < ntiles; it++) {
    const int64_t r0 = qstart + (int64_t)it * TILE;
    if (it > 0) __syncthreads();
    st.store(Qs, Qt, Os, Ot);
    if (threadIdx.x < TILE) {
      const int64_t qq = r0 + threadIdx.x;
      Ls[threadIdx.x] = qq < t_q ? lse[b * t_q + qq] * LOG2E : 0.f;
      Ds[threadIdx.x] = qq < t_q ? delta[b * t_q + qq] : 0.f;
    }
    __syncthreads();
    if (it + 1 < ntiles) st.load(qbase, obase, r0 + TILE, t_q);
    if (CAUSAL && r0 + TILE - 1 < wk0) continue;  // every query of this tile is left of this wave's keys

    f32x16 s[2], dp[2];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      s[sub] = zero16();
      dp[sub] = zero16();
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++) {
        const u16x8 a = *(const u16x8*)(Qs + (sub * 32 + n) * RS + ds * 16 + 8 * h);
        s[sub] = T::mfma32(a, kf[ds], s[sub]);
        const u16x8 e = *(const u16x8*)(Os + (sub * 32 + n) * RS + ds * 16 + 8 * h);
        dp[sub] = T::mfma32(e, vf[ds], dp[sub]);
      }
    }
    const bool edge = (r0 + TILE > t_q) || MASK || (CAUSAL && r0 < wk0 + 31);
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int rb = sub * 32 + 8 * g + 4 * h;
        const f32x4 l4 = *(const f32x4*)(Ls + rb);
        const f32x4 d4 = *(const f32x4*)(Ds + rb);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int i = 4 * g + e;
          float p = fast_exp2(fmaf(s[sub][i], c2, -l4[e]));
          if (edge) {
            const int64_t qq = r0 + rb + e;
            const bool hide = qq >= t_q || (CAUSAL && qq < key) || !live;
            if (hide) p = 0.f;
          }
          s[sub][i] = p;
          dp[sub][i] = p * (dp[sub][i] - d4[e]) * scale;
        }
      }
#pragma unroll
    for (int sub = 0; sub < 2; sub++)
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 pb, gb;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          pb[j] = T::pack(s[sub][8 * c + j]);
          gb[j] = T::pack(dp[sub][8 * c + j]);
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          const int d = dt * 32 + n, pos = trot(d, sub * 32 + 16 * c + 8 * h);
          const u16x8 a = *(const u16x8*)(Ot + d * CS + pos);
          gv[dt] = T::mfma32(a, pb, gv[dt]);
          const u16x8 e = *(const u16x8*)(Qt + d * CS + pos);
          gk[dt] = T::mfma32(e, gb, gk[dt]);
        }
      }
  }
  store_transposed<T, D>(dk + b * t_k * D, gk, key, t_k, 1.f);
  store_transposed<T, D>(dv + b * t_k * D, gv, key, t_k, 1.f);
}

// ---------------------------------------------------------------------------------------------

template <typename T, int D, bool CAUSAL, bool MASK>
int launch(SdpaPass pass, const SdpaArgs& a) {
  const int64_t rows = pass == SDPA_BWD_KV ? a.t_k : a.t_q;
  const int64_t blocks = a.batch * ((rows + BLOCK_ROWS - 1) / BLOCK_ROWS);
  if (blocks > 0x7fffffff) return fail(LIMN_HIP_EUNSUPPORTED, "sdpa: %lld workgroups exceed one launch", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(THREADS);
  const float scale = (float)a.scale;
  const u16* mask = (const u16*)a.mask;
  switch (pass) {
    case SDPA_FWD:
      hipLaunchKernelGGL((sdpa_fwd_mfma<T, D, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                         (const u16*)a.k, (const u16*)a.v, mask, (u16*)a.out0, (float*)a.out1, a.batch, a.t_q, a.t_k,
                         scale);
      break;
    case SDPA_BWD_Q:
      hipLaunchKernelGGL((sdpa_bwd_q_mfma<T, D, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                         (const u16*)a.k, (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse,
                         (const float*)a.delta, mask, (u16*)a.out0, a.batch, a.t_q, a.t_k, scale);
      break;
    case SDPA_BWD_KV:
      hipLaunchKernelGGL((sdpa_bwd_kv_mfma<T, D, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                         (const u16*)a.k, (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse,
                         (const float*)a.delta, mask, (u16*)a.out0, (u16*)a.out1, a.batch, a.t_q, a.t_k, scale);
      break;
  }
  return check_hip(hipGetLastError(), "launching an sdpa kernel");
}

template <typename T, int D>
int launch_flags(SdpaPass pass, const SdpaArgs& a) {
  const bool masked = a.mask != nullptr;
  if (a.causal) return masked ? launch<T, D, true, true>(pass, a) : launch<T, D, true, false>(pass, a);
  return masked ? launch<T, D, false, true>(pass, a) : launch<T, D, false, false>(pass, a);
}

template <typename T>
int launch_dim(SdpaPass pass, const SdpaArgs& a) {
  if (a.hd == 64) return launch_flags<T, 64>(pass, a);
  return launch_flags<T, 128>(pass, a);
}

}  // namespace

bool mfma_supports(int dtype, int64_t hd, int64_t hd_v) {
  return (dtype == LIMN_HIP_BFLOAT16 || dtype == LIMN_HIP_FLOAT16) && hd == hd_v && (hd == 64 || hd == 128);
}

int launch_sdpa_mfma(SdpaPass pass, const SdpaArgs& a) {
  if (a.dtype == LIMN_HIP_BFLOAT16) return launch_dim<BF16>(pass, a);
  return launch_dim<F16>(pass, a);
}

}  // namespace limn
