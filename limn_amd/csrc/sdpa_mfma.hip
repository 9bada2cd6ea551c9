// Flash attention on CDNA4 matrix cores: bf16/f16 storage, f32 accumulation and softmax
// statistics, head dim D in {64, 128} (hd == hd_v). Forward, dQ pass and dK/dV pass, the
// three CUSTOM kernels limn's attention seam asks for (reference limn/tensor.py:509-575,
// 679-714), each deterministic: every total is accumulated inside one wave in a fixed order.
//
// Work decomposition (all three kernels):
//   a workgroup is 4 waves and owns 128 * NT *resident* rows (queries for the forward and dQ
//   pass, keys for the dK/dV pass), NT tiles of 32 per wave; the other side *streams* past in
//   tiles of TILE = 64 rows staged through LDS (the next tile's global loads in flight while the
//   current one is computed) and is consumed 32 streamed rows at a time. Each operand fragment
//   read from LDS feeds NT MFMAs, one per resident tile: at NT = 1 one 1 KB read per MFMA
//   would ask LDS for its full bandwidth just to keep the matrix cores fed.
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
constexpr int TILE = 64;
constexpr float LOG2E = 1.4426950408889634f;
// The forward lets probabilities reach 2^RESCALE_LOG2 before it moves a row's reference max.
constexpr float RESCALE_LOG2 = 8.f;

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }

// Position of streamed row r (0..TILE-1) in a transposed LDS tile: within each 32-row
// sub-tile the 4-row groups g = 4c + 2q + h are reordered to 4c + 2h + q, so the 8 rows
// {16c + 8q + 4h + e} that lane half h feeds to k-chunk c are contiguous at 16c + 8h.
__device__ __forceinline__ int tpos(int r) {
  const int g = (r >> 2) & 7;
  const int gp = (g & 4) | ((g & 1) << 1) | ((g >> 1) & 1);
  return (r & ~31) | (gp << 2) | (r & 3);
}

// A transposed tile's row `d` stores its TILE positions rotated by 8 * ((d >> 4) & 7).
// gfx950's LDS has 64 four-byte banks and serves 16 lanes of a 16-byte access (32 lanes of an
// 8-byte one) per cycle. The row stride of TILE + 8 elements is 36 banks, so the 16 consecutive
// rows an MFMA operand read touches per cycle start in 16 distinct 4-bank groups as long as they
// share a rotation, which rows 16-aligned do. A staging store (one 8-byte column piece per lane,
// rows 8 apart) would put every even and every odd row chunk on the same bank group; the
// rotation by row >> 4 spreads those 16 rows over the 16 groups, and `stage_group` gives the two
// 16-lane halves of each 32 lanes the row groups whose positions are 8 bytes apart, so together
// they fill all 64 banks.
__device__ __forceinline__ int trot(int d, int pos) { return (pos + 8 * ((d >> 4) & 7)) & (TILE - 1); }

// The 4-row group staged by the threads with group index j: bits 0 and 1 swapped, so lanes
// 0-15 and 16-31 of a wave carry groups 4i and 4i + 2, which tpos() puts 8 bytes apart.
__device__ __forceinline__ int stage_group(int j) { return (j & ~3) | ((j & 1) << 1) | ((j >> 1) & 1); }

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

// A (rows x D) row-major matrix of one head, read through a buffer resource: the hardware
// bounds check returns zeros for rows past the end, so loads need no branches.
struct Rows {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ __forceinline__ Rows(const u16* base, int rows, int width) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, rows * width * 2, 0x00020000);
  }
  // 8 elements starting at element `offset` (zeros when past the end)
  __device__ __forceinline__ u16x8 load8(int offset) const {
    return __builtin_bit_cast(u16x8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset * 2, 0, 0));
  }
};

// Global -> registers -> LDS staging of one or two TILE x D row-major tiles. Each participating
// thread carries a 4-row x 8-column block, so it can write its rows (16 B per row) into a
// row-major LDS tile and its columns (8 B per column, 4 rows) into a transposed one.
template <int D>
struct Stage {
  static constexpr int COLS = D / 8;           // 16-byte column chunks per row
  static constexpr int PER_TILE = COLS * (TILE / 4);
  static constexpr int SLOTS = (2 * PER_TILE + THREADS - 1) / THREADS;  // both tiles
  u16x8 r[SLOTS][4];

  // rows [row0, row0 + TILE) of both matrices; rows past their end read as zeros
  __device__ __forceinline__ void load(const Rows& m0, const Rows& m1, int row0) {
#pragma unroll
    for (int s = 0; s < SLOTS; s++) {
      const int idx = threadIdx.x + s * THREADS;
      if (idx < 2 * PER_TILE) {
        const int which = idx / PER_TILE, w = idx - which * PER_TILE;
        const int col = w % COLS, grp = stage_group(w / COLS);
        const Rows& m = which ? m1 : m0;
#pragma unroll
        for (int e = 0; e < 4; e++) r[s][e] = m.load8((row0 + grp * 4 + e) * D + col * 8);
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
        const int col = w % COLS, grp = stage_group(w / COLS);
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
__device__ __forceinline__ void store_transposed(u16* base, const f32x16* acc, int row, int rows, float mul) {
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

// One batch row of the key mask, read through a buffer resource: entries past t_k read as zero,
// which is "hidden", so the last tile needs no bounds test.
struct MaskRow {
  __amdgpu_buffer_rsrc_t rsrc;
  __device__ __forceinline__ MaskRow(const u16* base, int t_k) {
    rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, t_k * 2, 0x00020000);
  }
  __device__ __forceinline__ u16 load(int key) const { return __builtin_amdgcn_raw_buffer_load_b16(rsrc, key * 2, 0, 0); }
};

// The live keys of a 64-key tile as one wave-uniform 64-bit word (bit r = key k0 + r is visible):
// each lane holds the mask entry of key k0 + lane, one 2-byte load per lane per tile, issued a
// tile ahead. Nothing of the mask goes through LDS or holds vector registers across the tile.
template <typename T>
__device__ __forceinline__ uint64_t live_keys(u16 entry) {
  return __ballot(T::unpack(entry) != 0.f);
}

// Whether accumulator item i of a 32-key half is a key that `row` may not see: past t_k, right of
// the row under a causal mask, or zero in the key mask (`mb` = the tile's live-key word shifted
// to the lane's first key, sub * 32 + 4 * h). Bitwise terms applied by the callers as selects: a
// short-circuit form, whose mask read sat under a branch, was compiled into code that left item 0
// visible whatever its mask said.
template <bool CAUSAL, bool MASK>
__device__ __forceinline__ bool hidden(int k0, int sub, int i, int h, int t_k, int row, unsigned mb) {
  const int key = k0 + sub * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
  bool hide = key >= t_k;
  if (CAUSAL) hide |= key > row;
  if (MASK) hide |= ((mb >> (8 * (i >> 2) + (i & 3))) & 1u) == 0u;
  return hide;
}

// ---------------------------------------------------------------------------------------------
// Forward. NT 32-row query tiles per wave: every K or V^T fragment read from LDS feeds NT MFMAs.
// The 64-key streamed tile is taken 32 keys at a time, one online-softmax step each. A causal
// half that lies wholly right of a wave's rows is computed anyway and masked to exact zeros:
// skipping it would branch around the accumulators, and the register allocator answers such a
// join by copying every accumulator register.
template <typename T, int D, int NT, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, NT == 1 ? 2 : 1) void sdpa_fwd_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                            const u16* __restrict__ v, const u16* __restrict__ mask,
                                                            u16* __restrict__ out, float* __restrict__ lse, int64_t batch,
                                                            int t_q, int t_k, float scale) {
  constexpr int RS = D + 8, CS = TILE + 8, ROWS = 128 * NT;
  __shared__ __attribute__((aligned(16))) u16 Ks[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Vt[D * CS];

  // the wave index in a scalar register: the per-wave tile bounds and causal tests below are then
  // uniform branches instead of exec-masked ones
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + ROWS - 1) / ROWS;
  const int64_t b = blockIdx.x % batch;
  const int64_t qb = nqb - 1 - blockIdx.x / batch;  // causal: the longest rows go first
  const int q0 = (int)qb * ROWS, wq0 = q0 + wave * 32 * NT;
  const Rows qrows(q + b * (int64_t)t_q * D, t_q, D);
  const Rows krows(k + b * (int64_t)t_k * D, t_k, D), vrows(v + b * (int64_t)t_k * D, t_k, D);
  const float c2 = scale * LOG2E, lift = RESCALE_LOG2 / c2;  // scale > 0 (the C ABI routes others away)

  u16x8 qf[NT][D / 16];
  f32x16 acc[NT][D / 32];
  float m[NT], l[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int row = wq0 + 32 * t + n;
#pragma unroll
    for (int ds = 0; ds < D / 16; ds++) qf[t][ds] = qrows.load8(row * D + ds * 16 + 8 * h);
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) acc[t][dt] = zero16();
    m[t] = neg_inf();
    l[t] = 0.f;
  }

  const int kend = CAUSAL ? (q0 + ROWS < t_k ? q0 + ROWS : t_k) : t_k;
  const int ntiles = (kend + TILE - 1) / TILE;
  Stage<D> st;
  st.load(krows, vrows, 0);
  const MaskRow mrow(MASK ? mask + b * (int64_t)t_k : nullptr, t_k);
  u16 mnext = MASK ? mrow.load(lane) : (u16)0;
  for (int it = 0; it < ntiles; it++) {
    const int k0 = it * TILE;
    if (it > 0) __syncthreads();
    st.store(Ks, nullptr, nullptr, Vt);
    __syncthreads();
    if (it + 1 < ntiles) st.load(krows, vrows, k0 + TILE);
    uint64_t live = ~0ull;
    if (MASK) {
      live = live_keys<T>(mnext);
      if (it + 1 < ntiles) mnext = mrow.load(k0 + TILE + lane);
    }
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      const int s0 = k0 + sub * 32;
      // every K fragment of this half first, then the MFMA chain: the reads overlap each other
      u16x8 kfr[D / 16];
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++) kfr[ds] = *(const u16x8*)(Ks + (sub * 32 + n) * RS + ds * 16 + 8 * h);
      f32x16 s[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) s[t] = zero16();
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++)
#pragma unroll
        for (int t = 0; t < NT; t++) s[t] = T::mfma32(kfr[ds], qf[t][ds], s[t]);
      // a half needs masking when it runs past t_k, holds a hidden key, or crosses the diagonal
      const unsigned half_live = (unsigned)(live >> (sub * 32));
      const bool edge = (s0 + 32 > t_k) || (MASK && half_live != ~0u) || (CAUSAL && s0 + 31 > wq0);
      const unsigned mb = (unsigned)(live >> (sub * 32 + 4 * h));
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const int row = wq0 + 32 * t + n;
        if (edge) {
#pragma unroll
          for (int i = 0; i < 16; i++)
            s[t][i] = hidden<CAUSAL, MASK>(k0, sub, i, h, t_k, row, mb) ? neg_inf() : s[t][i];
        }
        float mx = neg_inf();
#pragma unroll
        for (int i = 0; i < 16; i++) mx = fmaxf(mx, s[t][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // m is the reference point of the row's exponentials, not its exact running max: it moves
        // (and the totals are rescaled) only when a half's max passes it by more than `lift`, i.e.
        // when some p would exceed 2^RESCALE_LOG2. Larger p are carried by the float totals and
        // the 16-bit P operands as exactly as p <= 1, and the D/2 multiplies per lane of the
        // rescale then run on the few halves whose max jumps, not on every half where some row's
        // max creeps up.
        if (__any(mx > m[t] + lift)) {
          const float mnew = fmaxf(m[t], mx);
          const float alpha = mnew == neg_inf() ? 1.f : fast_exp2((m[t] - mnew) * c2);
          l[t] *= alpha;
#pragma unroll
          for (int dt = 0; dt < D / 32; dt++) acc[t][dt] *= alpha;
          m[t] = mnew;
        }
        const float base = m[t] == neg_inf() ? 0.f : m[t] * c2;
        float rs = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const float p = fast_exp2(fmaf(s[t][i], c2, -base));
          s[t][i] = p;
          rs += p;
        }
        l[t] += rs;
      }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 vfr[D / 32];
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          const int d = dt * 32 + n;
          vfr[dt] = *(const u16x8*)(Vt + d * CS + trot(d, sub * 32 + 16 * c + 8 * h));
        }
        u16x8 pb[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) pb[t] = pack8<T>(s[t], 8 * c);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
          for (int t = 0; t < NT; t++) acc[t][dt] = T::mfma32(vfr[dt], pb[t], acc[t][dt]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int row = wq0 + 32 * t + n;
    const float total = l[t] + __shfl_xor(l[t], 32);
    store_transposed<T, D>(out + b * (int64_t)t_q * D, acc[t], row, t_q, 1.f / total);
    if (h == 0 && row < t_q) lse[b * (int64_t)t_q + row] = m[t] * scale + logf(total);
  }
}

// ---------------------------------------------------------------------------------------------
// dQ pass: resident query rows (NT tiles per wave), keys streaming 32 at a time.
template <typename T, int D, int NT, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 1) void sdpa_bwd_q_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                              const u16* __restrict__ v, const u16* __restrict__ dout,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ delta,
                                                              const u16* __restrict__ mask, u16* __restrict__ dq,
                                                              int64_t batch, int t_q, int t_k, float scale) {
  constexpr int RS = D + 8, CS = TILE + 8, ROWS = 128 * NT;
  __shared__ __attribute__((aligned(16))) u16 Ks[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Vs[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Kt[D * CS];

  // the wave index in a scalar register: the per-wave tile bounds and causal tests below are then
  // uniform branches instead of exec-masked ones
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + ROWS - 1) / ROWS;
  const int64_t b = blockIdx.x % batch;
  const int64_t qb = nqb - 1 - blockIdx.x / batch;
  const int q0 = (int)qb * ROWS, wq0 = q0 + wave * 32 * NT;
  const Rows qrows(q + b * (int64_t)t_q * D, t_q, D), orows(dout + b * (int64_t)t_q * D, t_q, D);
  const Rows krows(k + b * (int64_t)t_k * D, t_k, D), vrows(v + b * (int64_t)t_k * D, t_k, D);
  const float c2 = scale * LOG2E;

  u16x8 qf[NT][D / 16], of[NT][D / 16];
  f32x16 acc[NT][D / 32];
  float L2[NT], Dr[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int row = wq0 + 32 * t + n;
#pragma unroll
    for (int ds = 0; ds < D / 16; ds++) {
      qf[t][ds] = qrows.load8(row * D + ds * 16 + 8 * h);
      of[t][ds] = orows.load8(row * D + ds * 16 + 8 * h);
    }
    L2[t] = row < t_q ? lse[b * (int64_t)t_q + row] * LOG2E : 0.f;
    Dr[t] = row < t_q ? delta[b * (int64_t)t_q + row] : 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) acc[t][dt] = zero16();
  }

  const int kend = CAUSAL ? (q0 + ROWS < t_k ? q0 + ROWS : t_k) : t_k;
  const int ntiles = (kend + TILE - 1) / TILE;
  Stage<D> st;
  st.load(krows, vrows, 0);
  const MaskRow mrow(MASK ? mask + b * (int64_t)t_k : nullptr, t_k);
  u16 mnext = MASK ? mrow.load(lane) : (u16)0;
  for (int it = 0; it < ntiles; it++) {
    const int k0 = it * TILE;
    if (it > 0) __syncthreads();
    st.store(Ks, Kt, Vs, nullptr);
    __syncthreads();
    if (it + 1 < ntiles) st.load(krows, vrows, k0 + TILE);
    uint64_t live = ~0ull;
    if (MASK) {
      live = live_keys<T>(mnext);
      if (it + 1 < ntiles) mnext = mrow.load(k0 + TILE + lane);
    }
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      const int s0 = k0 + sub * 32;
      f32x16 s[NT], dp[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        s[t] = zero16();
        dp[t] = zero16();
      }
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++) {
        const u16x8 a = *(const u16x8*)(Ks + (sub * 32 + n) * RS + ds * 16 + 8 * h);
        const u16x8 e = *(const u16x8*)(Vs + (sub * 32 + n) * RS + ds * 16 + 8 * h);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          s[t] = T::mfma32(a, qf[t][ds], s[t]);
          dp[t] = T::mfma32(e, of[t][ds], dp[t]);
        }
      }
      // a half needs masking when it runs past t_k, holds a hidden key, or crosses the diagonal
      const unsigned half_live = (unsigned)(live >> (sub * 32));
      const bool edge = (s0 + 32 > t_k) || (MASK && half_live != ~0u) || (CAUSAL && s0 + 31 > wq0);
      const unsigned mb = (unsigned)(live >> (sub * 32 + 4 * h));
#pragma unroll
      for (int t = 0; t < NT; t++) {
        const int row = wq0 + 32 * t + n;
#pragma unroll
        for (int i = 0; i < 16; i++) {
          float p = fast_exp2(fmaf(s[t][i], c2, -L2[t]));
          if (edge) p = hidden<CAUSAL, MASK>(k0, sub, i, h, t_k, row, mb) ? 0.f : p;
          s[t][i] = p * (dp[t][i] - Dr[t]) * scale;
        }
      }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 g[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) g[t] = pack8<T>(s[t], 8 * c);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          const int d = dt * 32 + n;
          const u16x8 a = *(const u16x8*)(Kt + d * CS + trot(d, sub * 32 + 16 * c + 8 * h));
#pragma unroll
          for (int t = 0; t < NT; t++) acc[t][dt] = T::mfma32(a, g[t], acc[t][dt]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) store_transposed<T, D>(dq + b * (int64_t)t_q * D, acc[t], wq0 + 32 * t + n, t_q, 1.f);
}

// ---------------------------------------------------------------------------------------------
// dK/dV pass: resident key rows (NT tiles per wave), queries streaming 32 at a time.
template <typename T, int D, int NT, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 1) void sdpa_bwd_kv_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                               const u16* __restrict__ v, const u16* __restrict__ dout,
                                                               const float* __restrict__ lse,
                                                               const float* __restrict__ delta,
                                                               const u16* __restrict__ mask, u16* __restrict__ dk,
                                                               u16* __restrict__ dv, int64_t batch, int t_q,
                                                               int t_k, float scale) {
  constexpr int RS = D + 8, CS = TILE + 8, ROWS = 128 * NT;
  __shared__ __attribute__((aligned(16))) u16 Qs[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Os[TILE * RS];
  __shared__ __attribute__((aligned(16))) u16 Qt[D * CS];
  __shared__ __attribute__((aligned(16))) u16 Ot[D * CS];
  __shared__ __attribute__((aligned(16))) float Ls[TILE];
  __shared__ __attribute__((aligned(16))) float Ds[TILE];

  // the wave index in a scalar register: the per-wave tile bounds and causal tests below are then
  // uniform branches instead of exec-masked ones
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int64_t b = blockIdx.x % batch;
  const int64_t kb = blockIdx.x / batch;  // causal: the first keys are seen by the most queries
  const int k0 = (int)kb * ROWS, wk0 = k0 + wave * 32 * NT;
  const Rows qrows(q + b * (int64_t)t_q * D, t_q, D), orows(dout + b * (int64_t)t_q * D, t_q, D);
  const Rows krows(k + b * (int64_t)t_k * D, t_k, D), vrows(v + b * (int64_t)t_k * D, t_k, D);
  const float c2 = scale * LOG2E;

  u16x8 kf[NT][D / 16], vf[NT][D / 16];
  f32x16 gk[NT][D / 32], gv[NT][D / 32];
  bool live[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int key = wk0 + 32 * t + n;
#pragma unroll
    for (int ds = 0; ds < D / 16; ds++) {
      kf[t][ds] = krows.load8(key * D + ds * 16 + 8 * h);
      vf[t][ds] = vrows.load8(key * D + ds * 16 + 8 * h);
    }
    live[t] = key < t_k;
    if (MASK) live[t] = live[t] & (T::unpack(mask[b * (int64_t)t_k + (key < t_k ? key : t_k - 1)]) != 0.f);
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) {
      gk[t][dt] = zero16();
      gv[t][dt] = zero16();
    }
  }

  const int qstart = CAUSAL ? k0 : 0;  // a causal key is seen by queries at or after it
  const int ntiles = qstart < t_q ? (t_q - qstart + TILE - 1) / TILE : 0;
  Stage<D> st;
  if (ntiles > 0) st.load(qrows, orows, qstart);
  for (int it = 0; it < ntiles; it++) {
    const int r0 = qstart + it * TILE;
    if (it > 0) __syncthreads();
    st.store(Qs, Qt, Os, Ot);
    if (threadIdx.x < TILE) {
      const int qq = r0 + threadIdx.x;
      Ls[threadIdx.x] = qq < t_q ? lse[b * (int64_t)t_q + qq] * LOG2E : 0.f;
      Ds[threadIdx.x] = qq < t_q ? delta[b * (int64_t)t_q + qq] : 0.f;
    }
    __syncthreads();
    if (it + 1 < ntiles) st.load(qrows, orows, r0 + TILE);
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      const int s0 = r0 + sub * 32;
      f32x16 s[NT], dp[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        s[t] = zero16();
        dp[t] = zero16();
      }
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++) {
        const u16x8 a = *(const u16x8*)(Qs + (sub * 32 + n) * RS + ds * 16 + 8 * h);
        const u16x8 e = *(const u16x8*)(Os + (sub * 32 + n) * RS + ds * 16 + 8 * h);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          s[t] = T::mfma32(a, kf[t][ds], s[t]);
          dp[t] = T::mfma32(e, vf[t][ds], dp[t]);
        }
      }
      const bool edge = (s0 + 32 > t_q) || MASK || (CAUSAL && s0 < wk0 + 32 * NT - 1);
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int rb = sub * 32 + 8 * g + 4 * h;
        const f32x4 l4 = *(const f32x4*)(Ls + rb);
        const f32x4 d4 = *(const f32x4*)(Ds + rb);
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const int key = wk0 + 32 * t + n;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int i = 4 * g + e;
            float p = fast_exp2(fmaf(s[t][i], c2, -l4[e]));
            if (edge) {
              const int qq = r0 + rb + e;
              bool hide = (qq >= t_q) | !live[t];
              if (CAUSAL) hide |= qq < key;
              p = hide ? 0.f : p;
            }
            s[t][i] = p;
            dp[t][i] = p * (dp[t][i] - d4[e]) * scale;
          }
        }
      }
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 pb[NT], gb[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
          pb[t] = pack8<T>(s[t], 8 * c);
          gb[t] = pack8<T>(dp[t], 8 * c);
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          const int d = dt * 32 + n, pos = trot(d, sub * 32 + 16 * c + 8 * h);
          const u16x8 a = *(const u16x8*)(Ot + d * CS + pos);
          const u16x8 e = *(const u16x8*)(Qt + d * CS + pos);
#pragma unroll
          for (int t = 0; t < NT; t++) {
            gv[t][dt] = T::mfma32(a, pb[t], gv[t][dt]);
            gk[t][dt] = T::mfma32(e, gb[t], gk[t][dt]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int key = wk0 + 32 * t + n;
    store_transposed<T, D>(dk + b * (int64_t)t_k * D, gk[t], key, t_k, 1.f);
    store_transposed<T, D>(dv + b * (int64_t)t_k * D, gv[t], key, t_k, 1.f);
  }
}

// ---------------------------------------------------------------------------------------------

// Resident 32-row tiles per wave for each pass and head dim: 2 (each LDS operand read feeds two
// MFMAs) wherever the accumulators still fit the register file.
template <int D>
constexpr int tiles_per_wave(SdpaPass pass) {
  if (pass == SDPA_FWD) return 1;  // two workgroups per CU hide its latency better than operand reuse
  return (pass == SDPA_BWD_KV && D == 128) ? 1 : 2;
}

template <typename T, int D, int NT, bool CAUSAL, bool MASK, SdpaPass PASS>
int launch_nt(const SdpaArgs& a) {
  constexpr SdpaPass pass = PASS;
  const int64_t rows = pass == SDPA_BWD_KV ? a.t_k : a.t_q;
  const int64_t per = 128 * NT;
  const int64_t blocks = a.batch * ((rows + per - 1) / per);
  if (blocks > 0x7fffffff) return fail(LIMN_HIP_EUNSUPPORTED, "sdpa: %lld workgroups exceed one launch", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(THREADS);
  const float scale = (float)a.scale;
  const u16* mask = (const u16*)a.mask;
  if constexpr (PASS == SDPA_FWD) {
    hipLaunchKernelGGL((sdpa_fwd_mfma<T, D, NT, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                       (const u16*)a.k, (const u16*)a.v, mask, (u16*)a.out0, (float*)a.out1, a.batch, (int)a.t_q, (int)a.t_k,
                       scale);
  } else if constexpr (PASS == SDPA_BWD_Q) {
    hipLaunchKernelGGL((sdpa_bwd_q_mfma<T, D, NT, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                       (const u16*)a.k, (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse, (const float*)a.delta,
                       mask, (u16*)a.out0, a.batch, (int)a.t_q, (int)a.t_k, scale);
  } else {
    hipLaunchKernelGGL((sdpa_bwd_kv_mfma<T, D, NT, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                       (const u16*)a.k, (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse, (const float*)a.delta,
                       mask, (u16*)a.out0, (u16*)a.out1, a.batch, (int)a.t_q, (int)a.t_k, scale);
  }
  return check_hip(hipGetLastError(), "launching an sdpa kernel");
}

template <typename T, int D, bool CAUSAL, bool MASK>
int launch(SdpaPass pass, const SdpaArgs& a) {
  switch (pass) {
    case SDPA_FWD:
      return launch_nt<T, D, tiles_per_wave<D>(SDPA_FWD), CAUSAL, MASK, SDPA_FWD>(a);
    case SDPA_BWD_Q:
      return launch_nt<T, D, tiles_per_wave<D>(SDPA_BWD_Q), CAUSAL, MASK, SDPA_BWD_Q>(a);
    default:
      return launch_nt<T, D, tiles_per_wave<D>(SDPA_BWD_KV), CAUSAL, MASK, SDPA_BWD_KV>(a);
  }
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

bool mfma_fits(int64_t t_q, int64_t t_k, int64_t hd) {
  // per-head offsets are 32-bit inside the kernels
  const int64_t limit = ((int64_t)1 << 31) - 1;
  return t_q * hd < limit && t_k * hd < limit;
}

int launch_sdpa_mfma(SdpaPass pass, const SdpaArgs& a) {
  if (a.dtype == LIMN_HIP_BFLOAT16) return launch_dim<BF16>(pass, a);
  return launch_dim<F16>(pass, a);
}

}  // namespace limn
