// Flash attention on CDNA4 matrix cores: bf16/f16 storage, f32 accumulation and softmax
// statistics, head dim D in {64, 128} (hd == hd_v). Forward, dQ pass and dK/dV pass, the
// three CUSTOM kernels limn's attention seam asks for (reference limn/tensor.py:509-575,
// 679-714), each deterministic: every total is accumulated inside one wave in a fixed order.
//
// Work decomposition (all three kernels; the unmasked D = 128 dK/dV pass differs, see
// sdpa_bwd_kv_dual):
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
// is the streamed operand transposed: it is read from the same row-major LDS tile with gfx950's
// transposing LDS read (ds_read_b64_tr_b16), addressed so that lane l gets exactly those 8 rows.
//
// LDS: each streamed tile is stored once, row-major with padded, permuted rows (tile_row), and
// double-buffered: the next tile is written into the other buffer as soon as a wave finishes the
// current one, behind one barrier per tile.
//
// 32x32 accumulator layout (CDNA3/CDNA4 matrix cores): lane l, item i holds
// row 8*(i/4) + 4*(l/32) + i%4, column l%32.
//
// This header holds every kernel and launch template with internal linkage; each sdpa_mfma_*.hip
// translation unit instantiates one pass (they compile in parallel), sdpa_mfma.hip dispatches.

#pragma once

#include <type_traits>

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

// x combined with the same register of lane ^ 32 (the other half of a row's 32x32 accumulator
// column), through gfx950's v_permlane32_swap: a VALU exchange instead of an LDS permute. The
// swap trades the upper half of its first operand with the lower half of its second; given x
// twice, it returns x from lane & 31 and from 32 + (lane & 31), so both lanes of a row combine
// the same two values. Replacing __shfl_xor(x, 32) here took the D = 128 forward from 0.640 to
// 0.587 ms at 128 heads x 4096 rows, causal, with identical results.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

// The (head, row block) a workgroup owns. Workgroup id runs on XCD id % 8: each XCD is given a
// contiguous run of ids covering groups of HEAD_GROUP heads, so a group's blocks run together on
// one XCD and share its L2's copy of the streamed operands (4 MB of L2 per XCD; a head's K and V,
// or Q and dO, are 2 MB at t = 4096, D = 128). Within a group the ids go block-major, the heads
// alternating, and the kernels number blocks so that the longest (under causal) go first: the
// XCD then starts its longest blocks early, where heads one after another would leave the last
// head's longest block to start near the end. Measured on the MI355X at 128 heads x 4096 rows,
// causal: the forward took 0.604 ms with whole heads in order, 0.569 with pairs, 0.548 with
// groups of 4 or 8, 0.554 with 16. The dQ pass from the handed-over dS takes groups of 8: 0.464
// against 0.482 ms with 4, alternating builds on one box (0.459-0.464 with 16, 0.62 with 32).
constexpr int HEAD_GROUP = 4;
constexpr int DQ_HEAD_GROUP = 8;

// Work units of the D = 64 passes per head: under causality a block and its mirror (the block
// counted from the other end) make one unit, so every unit walks the same number of tiles. At
// short sequences every workgroup is resident at once, and unpaired the longest blocks ran on
// alone at the end while the shorter ones had finished.
template <bool CAUSAL>
__host__ __device__ constexpr int64_t paired_units(int64_t blocks) {
  return CAUSAL ? (blocks + 1) / 2 : blocks;
}

template <int G = HEAD_GROUP>
__device__ __forceinline__ void head_and_block(int64_t batch, int64_t nblocks, int64_t& b, int64_t& blk) {
  if (gridDim.x % 8 == 0) {
    const int64_t id = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
    const int64_t group = id / (G * nblocks), r = id % (G * nblocks);
    const int64_t heads = batch - G * group < G ? batch - G * group : G;
    b = G * group + r % heads;
    blk = r / heads;
  } else {
    b = blockIdx.x % batch;
    blk = blockIdx.x / batch;
  }
}

// ---- LDS tiles -------------------------------------------------------------------------------
// A streamed tile is TILE rows x D elements, rows padded to D + 8 elements (a 16-byte chunk more
// than a multiple of 256 bytes, so consecutive physical rows start one 16-byte bank group apart),
// with the streamed rows permuted: row 4q + j of each 32 is stored at physical row
// (q >> 1) + 4j + 16 parity(q). gfx950's LDS has 64 banks of 4 bytes; measured on the MI355X, a
// 16-byte read is served 16 lanes per cycle, the lanes of each 32-lane half grouped by the parity
// of their quad index (lane >> 2) & 7; a transposing 8-byte read 32 lanes per cycle; a 16-byte
// write 8 consecutive lanes per cycle. Against that the layout makes every access conflict-free:
//   row operand reads (the 16 rows of one parity group, one chunk): the two quads q of a group
//     with equal q >> 1 sit 16 physical rows apart, so the 16 rows start in 16 different groups;
//   transposing reads (the 4 rows of an aligned quad, 4 chunks each): 4 physical rows apart, so
//     their 64-byte windows tile the 256-byte bank line;
//   staging writes (8 chunks of one row): contiguous.
// Every address is a per-lane base plus a compile-time offset, so reads cost no address VALU.
template <int D>
constexpr int tile_stride() { return D + 8; }

__device__ __forceinline__ int tile_row(int r) {
  const int q = (r >> 2) & 7;
  const int odd = (q ^ (q >> 1) ^ (q >> 2)) & 1;
  return (r & ~31) | ((q >> 1) + 4 * (r & 3) + 16 * odd);
}

// Element offset of element d of streamed row r.
template <int D>
__device__ __forceinline__ int tile_at(int r, int d) {
  return tile_row(r) * tile_stride<D>() + d;
}

// Row operand: elements 8c .. 8c + 7 of streamed row r, one ds_read_b128.
template <int D>
__device__ __forceinline__ u16x8 read_row(const u16* tile, int r, int c) {
  return *(const u16x8*)(tile + tile_at<D>(r, 8 * c));
}

// Transposed operand: lane l gets X[k0 + 4 (l / 32) + 8 (j / 4) + j % 4][d0 + l % 32], j = 0..7,
// of the tile X: the 8 streamed rows that items 8c..8c+7 of a lane's accumulator cover when
// k0 = 16c, which is what pack8 turns into the B operand. Two ds_read_b64_tr_b16 (j / 4 = 0, 1):
// within each 16-lane group, lane i receives item j' from the 8 bytes addressed by lane
// 4 j' + i / 4, element i % 4; so lane r of the group addresses row k0 + 4 (l / 32) + 8 (j / 4) +
// r / 4, columns d0 + 16 ((l / 16) % 2) + 4 (r % 4) .. + 3.
template <int D>
__device__ __forceinline__ u16x8 read_transposed(const u16* tile, int k0, int d0) {
  const int lane = threadIdx.x & 63, g = lane >> 4, i = lane & 15;
  const int d = d0 + 16 * (g & 1) + 4 * (i & 3);
  const int r = k0 + 4 * (g >> 1) + (i >> 2);
  u16* base = (u16*)tile;
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + tile_at<D>(r, d)));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(base + tile_at<D>(r + 8, d)));
  return __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

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

// Global -> registers -> LDS staging of two TILE x D row-major tiles. Each participating thread
// carries one 16-byte column chunk of 4 consecutive rows; 8 consecutive lanes write 8 chunks of
// one row.
template <int D>
struct Stage {
  static constexpr int COLS = D / 8;                  // 16-byte chunks per row
  static constexpr int PER_TILE = COLS * (TILE / 4);  // (chunk, 4-row group) blocks per tile
  static constexpr int SLOTS = (2 * PER_TILE + THREADS - 1) / THREADS;
  u16x8 r[SLOTS][4];

  static_assert(PER_TILE % 64 == 0, "a wave's blocks come from one matrix");

  // rows [row0, row0 + TILE) of both matrices; rows past their end read as zeros
  __device__ __forceinline__ void load(const Rows& m0, const Rows& m1, int row0) {
#pragma unroll
    for (int s = 0; s < SLOTS; s++) {
      const int idx = threadIdx.x + s * THREADS;
      if (idx < 2 * PER_TILE) {
        // a whole wave reads one matrix: saying so keeps its buffer resource in scalar
        // registers (a per-lane choice would wrap every load in a loop over distinct resources)
        const int which = __builtin_amdgcn_readfirstlane(idx / PER_TILE), w = idx - which * PER_TILE;
        const int col = w % COLS, grp = w / COLS;
        const Rows& m = which ? m1 : m0;
#pragma unroll
        for (int e = 0; e < 4; e++) r[s][e] = m.load8((row0 + grp * 4 + e) * D + col * 8);
      }
    }
  }

  __device__ __forceinline__ void store(u16* tile0, u16* tile1) {
#pragma unroll
    for (int s = 0; s < SLOTS; s++) {
      const int idx = threadIdx.x + s * THREADS;
      if (idx < 2 * PER_TILE) {
        const int which = idx / PER_TILE, w = idx - which * PER_TILE;
        const int col = w % COLS, grp = w / COLS;
        u16* tile = which ? tile1 : tile0;
#pragma unroll
        for (int e = 0; e < 4; e++) *(u16x8*)(tile + tile_at<D>(grp * 4 + e, col * 8)) = r[s][e];
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

// The wave's 32 rows x D dims of an accumulator set (lane n = row, items = dims, the layout
// store_transposed takes) to global rows [row0, row0 + 32) of a (rows x D) matrix, scaled by
// `mul`, through an LDS stage of 32 rows padded by 16 bytes: D / 8 8-byte LDS writes per lane,
// then 16-byte global stores each covering 512 / D whole rows. store_transposed's 8-byte stores
// touch 32 rows per instruction; staged, the D = 128 dK/dV pass took 1.143 ms against 1.194.
// The wave reads only what it wrote itself, so no barrier is needed between the two halves.
template <typename T, int D>
__device__ __forceinline__ void store_staged(u16* base, const f32x16* acc, int row0, int rows, float mul, u16* stage) {
  const int lane = threadIdx.x & 63, h = lane >> 5, n = lane & 31;
  constexpr int RS = D + 8;      // padded row stride, elements
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows one store instruction covers
#pragma unroll
  for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const u16x4 o = {T::pack(acc[dt][4 * g] * mul), T::pack(acc[dt][4 * g + 1] * mul), T::pack(acc[dt][4 * g + 2] * mul),
                       T::pack(acc[dt][4 * g + 3] * mul)};
      *(u16x4*)(stage + n * RS + dt * 32 + 8 * g + 4 * h) = o;
    }
#pragma unroll
  for (int j = 0; j < 32 / RPI; j++) {
    const int r = RPI * j + lane / CPR, c = lane % CPR;
    const u16x8 v = *(const u16x8*)(stage + r * RS + c * 8);
    if (row0 + r < rows) *(u16x8*)(base + (int64_t)(row0 + r) * D + c * 8) = v;
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
  constexpr int ROWS = 128 * NT;
  __shared__ __attribute__((aligned(16))) u16 Ks[2][TILE * tile_stride<D>()];
  __shared__ __attribute__((aligned(16))) u16 Vs[2][TILE * tile_stride<D>()];

  // the wave index in a scalar register: the per-wave tile bounds and causal tests below are then
  // uniform branches instead of exec-masked ones
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + ROWS - 1) / ROWS;
  // causal: a workgroup takes a block and its mirror, nqb - 1 - u then u, so that every
  // workgroup has the same work (see paired_units)
  const int64_t units = paired_units<CAUSAL>(nqb);
  int64_t b, unit;
  head_and_block(batch, units, b, unit);
  const int reps = CAUSAL && nqb - 1 - unit != unit ? 2 : 1;
#pragma unroll 1
  for (int rep = 0; rep < reps; rep++) {
  const int64_t qb = rep == 0 ? nqb - 1 - unit : unit;  // causal: the longest rows go first
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
  st.store(Ks[0], Vs[0]);
  if (ntiles > 1) st.load(krows, vrows, TILE);
  const MaskRow mrow(MASK ? mask + b * (int64_t)t_k : nullptr, t_k);
  u16 mnext = MASK ? mrow.load(lane) : (u16)0;
  __syncthreads();
  for (int it = 0; it < ntiles; it++) {
    const int k0 = it * TILE, buf = it & 1;
    const u16* Kt = Ks[buf];
    const u16* Vt = Vs[buf];
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
      for (int ds = 0; ds < D / 16; ds++) kfr[ds] = read_row<D>(Kt, sub * 32 + n, 2 * ds + h);
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
        mx = pair_max(mx);
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
        for (int dt = 0; dt < D / 32; dt++) vfr[dt] = read_transposed<D>(Vt, sub * 32 + 16 * c, dt * 32);
        u16x8 pb[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) pb[t] = pack8<T>(s[t], 8 * c);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
          for (int t = 0; t < NT; t++) acc[t][dt] = T::mfma32(vfr[dt], pb[t], acc[t][dt]);
      }
    }
    // the next tile into the other buffer (free since the last barrier), then the load after it
    if (it + 1 < ntiles) {
      st.store(Ks[buf ^ 1], Vs[buf ^ 1]);
      if (it + 2 < ntiles) st.load(krows, vrows, k0 + 2 * TILE);
    }
    __syncthreads();
  }
  __syncthreads();  // every wave is done with the tiles: each stages its output in one
  u16* stage = wave == 0 ? Ks[0] : wave == 1 ? Ks[1] : wave == 2 ? Vs[0] : Vs[1];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const int row = wq0 + 32 * t + n;
    const float total = pair_sum(l[t]);
    store_staged<T, D>(out + b * (int64_t)t_q * D, acc[t], wq0 + 32 * t, t_q, 1.f / total, stage);
    if (h == 0 && row < t_q) lse[b * (int64_t)t_q + row] = m[t] * scale + logf(total);
  }
    __syncthreads();  // the pair's second block reuses the LDS tiles
  }
}

// ---------------------------------------------------------------------------------------------
// dQ pass: resident query rows (NT tiles per wave), keys streaming 32 at a time.
template <typename T, int D, int NT, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, NT == 1 ? 2 : 1) void sdpa_bwd_q_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                              const u16* __restrict__ v, const u16* __restrict__ dout,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ delta,
                                                              const u16* __restrict__ mask, u16* __restrict__ dq,
                                                              int64_t batch, int t_q, int t_k, float scale) {
  constexpr int ROWS = 128 * NT;
  __shared__ __attribute__((aligned(16))) u16 Ks[2][TILE * tile_stride<D>()];
  __shared__ __attribute__((aligned(16))) u16 Vs[2][TILE * tile_stride<D>()];

  // the wave index in a scalar register: the per-wave tile bounds and causal tests below are then
  // uniform branches instead of exec-masked ones
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + ROWS - 1) / ROWS;
  // causal: a workgroup takes a block and its mirror, nqb - 1 - u then u, so that every
  // workgroup has the same work (see paired_units)
  const int64_t units = paired_units<CAUSAL>(nqb);
  int64_t b, unit;
  head_and_block(batch, units, b, unit);
  const int reps = CAUSAL && nqb - 1 - unit != unit ? 2 : 1;
#pragma unroll 1
  for (int rep = 0; rep < reps; rep++) {
  const int64_t qb = rep == 0 ? nqb - 1 - unit : unit;  // causal: the longest rows go first
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
    Dr[t] = row < t_q ? delta[b * (int64_t)t_q + row] * scale : 0.f;  // ds = p (dp scale - delta scale)
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) acc[t][dt] = zero16();
  }

  const int kend = CAUSAL ? (q0 + ROWS < t_k ? q0 + ROWS : t_k) : t_k;
  const int ntiles = (kend + TILE - 1) / TILE;
  Stage<D> st;
  st.load(krows, vrows, 0);
  st.store(Ks[0], Vs[0]);
  if (ntiles > 1) st.load(krows, vrows, TILE);
  const MaskRow mrow(MASK ? mask + b * (int64_t)t_k : nullptr, t_k);
  u16 mnext = MASK ? mrow.load(lane) : (u16)0;
  __syncthreads();
  for (int it = 0; it < ntiles; it++) {
    const int k0 = it * TILE, buf = it & 1;
    const u16* Kb = Ks[buf];
    const u16* Vb = Vs[buf];
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
        const u16x8 a = read_row<D>(Kb, sub * 32 + n, 2 * ds + h);
        const u16x8 e = read_row<D>(Vb, sub * 32 + n, 2 * ds + h);
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
      // the masking as one uniform block of selects (a test per item would be compiled into a
      // branch per item), then the probabilities, then dS. A hidden score is -inf, so its
      // probability exp2(-inf - L) is 0, or NaN in a row whose every key is hidden (L = -inf), as
      // in the numpy reference
      if (edge) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
          for (int i = 0; i < 16; i++) s[t][i] = hidden<CAUSAL, MASK>(k0, sub, i, h, t_k, wq0 + 32 * t + n, mb) ? neg_inf() : s[t][i];
      }
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) s[t][i] = fast_exp2(fmaf(s[t][i], c2, -L2[t]));
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) s[t][i] *= fmaf(dp[t][i], scale, -Dr[t]);
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 g[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) g[t] = pack8<T>(s[t], 8 * c);
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          const u16x8 a = read_transposed<D>(Kb, sub * 32 + 16 * c, dt * 32);
#pragma unroll
          for (int t = 0; t < NT; t++) acc[t][dt] = T::mfma32(a, g[t], acc[t][dt]);
        }
      }
    }
    if (it + 1 < ntiles) {
      st.store(Ks[buf ^ 1], Vs[buf ^ 1]);
      if (it + 2 < ntiles) st.load(krows, vrows, k0 + 2 * TILE);
    }
    __syncthreads();
  }
  __syncthreads();  // every wave is done with the tiles: each stages its output in one
  u16* stage = wave == 0 ? Ks[0] : wave == 1 ? Ks[1] : wave == 2 ? Vs[0] : Vs[1];
#pragma unroll
  for (int t = 0; t < NT; t++) store_staged<T, D>(dq + b * (int64_t)t_q * D, acc[t], wq0 + 32 * t, t_q, 1.f, stage);
    __syncthreads();  // the pair's second block reuses the LDS tiles
  }
}

// ---------------------------------------------------------------------------------------------
// dK/dV pass: resident key rows (NT tiles per wave), queries streaming 32 at a time.
template <typename T, int D, int NT, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, NT == 1 ? 2 : 1) void sdpa_bwd_kv_mfma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                               const u16* __restrict__ v, const u16* __restrict__ dout,
                                                               const float* __restrict__ lse,
                                                               const float* __restrict__ delta,
                                                               const u16* __restrict__ mask, u16* __restrict__ dk,
                                                               u16* __restrict__ dv, int64_t batch, int t_q,
                                                               int t_k, float scale) {
  constexpr int ROWS = 128 * NT;
  __shared__ __attribute__((aligned(16))) u16 Qs[2][TILE * tile_stride<D>()];
  __shared__ __attribute__((aligned(16))) u16 Os[2][TILE * tile_stride<D>()];
  __shared__ __attribute__((aligned(16))) float Ls[2][TILE];  // lse * log2(e) of the tile's queries
  __shared__ __attribute__((aligned(16))) float Ds[2][TILE];  // delta * scale

  // the wave index in a scalar register: the per-wave tile bounds and causal tests below are then
  // uniform branches instead of exec-masked ones
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  // causal: the first keys are seen by the most queries; a workgroup takes a key block and its
  // mirror, u then nkb - 1 - u (see paired_units)
  const int64_t nkb = (t_k + ROWS - 1) / ROWS, units = paired_units<CAUSAL>(nkb);
  int64_t b, unit;
  head_and_block(batch, units, b, unit);
  const int reps = CAUSAL && nkb - 1 - unit != unit ? 2 : 1;
#pragma unroll 1
  for (int rep = 0; rep < reps; rep++) {
  const int64_t kb = rep == 0 ? unit : nkb - 1 - unit;
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
  // the per-query statistics of a tile travel like its rows: loaded a tile ahead into registers
  // of the first wave, written into the tile's buffer with them
  auto stats_load = [&](int r0, float& ls, float& dl) {
    const int qq = r0 + (int)threadIdx.x;
    ls = qq < t_q ? lse[b * (int64_t)t_q + qq] * LOG2E : 0.f;
    dl = qq < t_q ? delta[b * (int64_t)t_q + qq] * scale : 0.f;
  };
  Stage<D> st;
  float lnext = 0.f, dnext = 0.f;
  if (ntiles > 0) {
    st.load(qrows, orows, qstart);
    if (threadIdx.x < TILE) stats_load(qstart, lnext, dnext);
    st.store(Qs[0], Os[0]);
    if (threadIdx.x < TILE) {
      Ls[0][threadIdx.x] = lnext;
      Ds[0][threadIdx.x] = dnext;
    }
    if (ntiles > 1) {
      st.load(qrows, orows, qstart + TILE);
      if (threadIdx.x < TILE) stats_load(qstart + TILE, lnext, dnext);
    }
  }
  __syncthreads();
  for (int it = 0; it < ntiles; it++) {
    const int r0 = qstart + it * TILE, buf = it & 1;
    const u16* Qb = Qs[buf];
    const u16* Ob = Os[buf];
    const float* Lb = Ls[buf];
    const float* Db = Ds[buf];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      const int s0 = r0 + sub * 32;
      f32x16 s[NT], dp[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        s[t] = zero16();
        dp[t] = zero16();
      }
      // one wave per SIMD: nothing else hides LDS latency, so every fragment of the half is read
      // before the MFMA chains that use them
      u16x8 qa[D / 16], oa[D / 16];
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++) {
        qa[ds] = read_row<D>(Qb, sub * 32 + n, 2 * ds + h);
        oa[ds] = read_row<D>(Ob, sub * 32 + n, 2 * ds + h);
      }
#pragma unroll
      for (int ds = 0; ds < D / 16; ds++)
#pragma unroll
        for (int t = 0; t < NT; t++) {
          s[t] = T::mfma32(qa[ds], kf[t][ds], s[t]);
          dp[t] = T::mfma32(oa[ds], vf[t][ds], dp[t]);
        }
      // the transposed fragments of both k-chunks, in flight during the softmax arithmetic
      u16x8 ot[2][D / 32], qt[2][D / 32];
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++) {
          ot[c][dt] = read_transposed<D>(Ob, sub * 32 + 16 * c, dt * 32);
          qt[c][dt] = read_transposed<D>(Qb, sub * 32 + 16 * c, dt * 32);
        }
      const bool edge = (s0 + 32 > t_q) || MASK || (CAUSAL && s0 < wk0 + 32 * NT - 1);
      // the statistics of the half's queries (item i <-> query rb(i / 4) + i % 4), the masking as
      // one uniform block of selects (a hidden score is -inf: probability 0, or NaN against a row
      // whose every key is hidden, as in the numpy reference), the probabilities, then dS
      f32x4 l4[4], d4[4];
#pragma unroll
      for (int g = 0; g < 4; g++) {
        l4[g] = *(const f32x4*)(Lb + sub * 32 + 8 * g + 4 * h);
        d4[g] = *(const f32x4*)(Db + sub * 32 + 8 * g + 4 * h);
      }
      if (edge) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
          const int key = wk0 + 32 * t + n;
#pragma unroll
          for (int i = 0; i < 16; i++) {
            const int qq = s0 + 8 * (i >> 2) + 4 * h + (i & 3);
            bool hide = (qq >= t_q) | !live[t];
            if (CAUSAL) hide |= qq < key;
            s[t][i] = hide ? neg_inf() : s[t][i];
          }
        }
      }
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) s[t][i] = fast_exp2(fmaf(s[t][i], c2, -l4[i >> 2][i & 3]));
#pragma unroll
      for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) dp[t][i] = s[t][i] * fmaf(dp[t][i], scale, -d4[i >> 2][i & 3]);
#pragma unroll
      for (int c = 0; c < 2; c++) {
        u16x8 pb[NT], gb[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
          pb[t] = pack8<T>(s[t], 8 * c);
          gb[t] = pack8<T>(dp[t], 8 * c);
        }
#pragma unroll
        for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
          for (int t = 0; t < NT; t++) {
            gv[t][dt] = T::mfma32(ot[c][dt], pb[t], gv[t][dt]);
            gk[t][dt] = T::mfma32(qt[c][dt], gb[t], gk[t][dt]);
          }
      }
    }
    if (it + 1 < ntiles) {
      st.store(Qs[buf ^ 1], Os[buf ^ 1]);
      if (threadIdx.x < TILE) {
        Ls[buf ^ 1][threadIdx.x] = lnext;
        Ds[buf ^ 1][threadIdx.x] = dnext;
      }
      if (it + 2 < ntiles) {
        st.load(qrows, orows, r0 + 2 * TILE);
        if (threadIdx.x < TILE) stats_load(r0 + 2 * TILE, lnext, dnext);
      }
    }
    __syncthreads();
  }
  __syncthreads();  // every wave is done with the tiles: each stages its output in one
  u16* stage = wave == 0 ? Qs[0] : wave == 1 ? Qs[1] : wave == 2 ? Os[0] : Os[1];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    store_staged<T, D>(dk + b * (int64_t)t_k * D, gk[t], wk0 + 32 * t, t_k, 1.f, stage);
    store_staged<T, D>(dv + b * (int64_t)t_k * D, gv[t], wk0 + 32 * t, t_k, 1.f, stage);
  }
    __syncthreads();  // the pair's second block reuses the LDS tiles
  }
}

// ---- dK/dV pass at D = 128: streamed tiles copied straight into LDS ----------------------------
// The streamed Q and dO tiles go from memory to LDS by buffer_load ... lds (no staging registers,
// no LDS write instructions), into unpadded tiles whose 16-byte chunk c of row r sits at position
// c ^ swz(r): lane-linear 1 KB DMA writes, and conflict-free row-operand and transposing reads
// (measured LDS model above). Each buffer is its own __shared__ array and tiles alternate between
// them in an unrolled pair, so the compiler sees that a copy into the idle buffer never aliases
// a read of the current one. The tiles that need masking (a causal wave's first two, holding
// every query before its last key, a last tile past t_q, every tile under a key mask) run a
// separate instance of the tile body from the unmasked ones, so each loop is one basic block
// whose LDS reads the scheduler can interleave with the MFMAs.

typedef __attribute__((address_space(3))) void lds_void;
constexpr int WAIT_VMEM = 0x0F70;  // s_waitcnt immediate: vmcnt(0), other counters free
// s_waitcnt immediate for vmcnt(n), n < 64, the other counters free: all but the n newest vector
// memory operations done. Vector memory operations (loads, LDS DMA copies and stores alike)
// retire in the order they were issued on this architecture, so this waits for everything issued
// before the n newest.
__host__ __device__ constexpr int wait_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
// cache policy of a buffer access (gfx940 family): nt, streamed past the caches. The dS hand-off
// is written once and read once, gigabytes a step; left cached, it evicts the re-read tiles.
constexpr int AUX_NT = 2;

__device__ __forceinline__ int swz128(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// rows [row0, row0 + TILE) of a (rows x 128) matrix into a swizzled tile, this wave's quarter
struct DmaTile128 {
  static constexpr int RB = 256, PASSES = TILE * RB / 1024 / WAVES;
  const char* base;
  int64_t bytes;
  int voff[PASSES];
  __device__ __forceinline__ DmaTile128(const u16* m, int rows, int wave, int lane) {
    base = (const char*)m;
    bytes = (int64_t)rows * RB;
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
      const int r = (p * WAVES + wave) * (1024 / RB) + lane / (RB / 16), pos = lane % (RB / 16);
      voff[p] = r * RB + ((pos ^ swz128(r)) * 16);
    }
  }
  // rows past the end read as zeros (the resource ends at the matrix)
  __device__ __forceinline__ void copy(u16* tile, int row0, int wave) const {
    const int64_t off = (int64_t)row0 * RB, left = bytes - off;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)(base + off), (short)0, (int)(left > 0 ? left : 0), 0x00020000);
#pragma unroll
    for (int p = 0; p < PASSES; p++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)((char*)tile + (p * WAVES + wave) * 1024), 16, voff[p], 0, 0, 0);
  }
};

// The same copy shared by the 8 waves of a two-waves-per-SIMD workgroup, this wave's eighth. (A
// separate struct: as a template over the wave count, hipcc's host pass dropped the launch stubs
// of the kernels that construct it.)
struct DmaTile128x8 {
  static constexpr int NW = 8, RB = 256, PASSES = TILE * RB / 1024 / NW;
  const char* base;
  int64_t bytes;
  int voff[PASSES];
  __device__ __forceinline__ DmaTile128x8(const u16* m, int rows, int wave, int lane) {
    base = (const char*)m;
    bytes = (int64_t)rows * RB;
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
      const int r = (p * NW + wave) * (1024 / RB) + lane / (RB / 16), pos = lane % (RB / 16);
      voff[p] = r * RB + ((pos ^ swz128(r)) * 16);
    }
  }
  // rows past the end read as zeros (the resource ends at the matrix)
  __device__ __forceinline__ void copy(u16* tile, int row0, int wave) const {
    const int64_t off = (int64_t)row0 * RB, left = bytes - off;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)(base + off), (short)0, (int)(left > 0 ? left : 0), 0x00020000);
#pragma unroll
    for (int p = 0; p < PASSES; p++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)((char*)tile + (p * NW + wave) * 1024), 16, voff[p], 0, 0, 0);
  }
};

// per-lane byte offsets into a swizzled tile: row operands (row n of a 32-row step, chunk 2 ds + h)
// by ds; transposing reads (rows 4 h + 8 jj + i / 4, columns 32 dt + 16 (g % 2) + 4 (i % 4)) by
// (dt, jj). Every read is then one of these plus a compile-time offset.
struct SwzReads128 {
  int row[8], tr[4][2];
  __device__ __forceinline__ SwzReads128(int lane) {
    const int n = lane & 31, h = lane >> 5, g = lane >> 4, i = lane & 15;
#pragma unroll
    for (int ds = 0; ds < 8; ds++) row[ds] = n * 256 + (((2 * ds + h) ^ swz128(n)) * 16);
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int jj = 0; jj < 2; jj++) {
        const int r = 4 * h + 8 * jj + (i >> 2), col = dt * 32 + 16 * (g & 1) + 4 * (i & 3);
        tr[dt][jj] = r * 256 + (((col >> 3) ^ swz128(r)) * 16) + (col & 7) * 2;
      }
  }
  // row operand: elements 16 ds + 8 h .. + 7 of row sub * 32 + n
  __device__ __forceinline__ u16x8 rows(const u16* tile, int sub, int ds) const {
    return *(const u16x8*)((const char*)tile + row[ds] + sub * 32 * 256);
  }
  // transposed operand of rows k0 .. k0 + 15, columns 32 dt .. + 31 (see read_transposed)
  __device__ __forceinline__ u16x8 transposed(const u16* tile, int k0, int dt) const {
    const char* p = (const char*)tile + k0 * 256;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + tr[dt][0]));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + tr[dt][1]));
    return __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

// one 64-query tile against the wave's 32 resident keys: per 32-query step, S = Q K^T and
// dP = dO V^T, the probabilities and dS, then dV^T += dO^T P and dK^T += Q^T dS
template <typename T, bool CAUSAL, bool MASK, bool EDGE>
__device__ __forceinline__ void kv_tile128(const u16* Qb, const u16* Ob, const float* Lb, const float* Db,
                                           const SwzReads128& ad, int r0, int wk0, int t_q, float c2, float scale,
                                           bool live, const u16x8 (&kf)[8], const u16x8 (&vf)[8], f32x16 (&gk)[4],
                                           f32x16 (&gv)[4]) {
  const int lane = threadIdx.x & 63, h = lane >> 5, n = lane & 31;
#pragma unroll
  for (int sub = 0; sub < 2; sub++) {
    const int s0 = r0 + sub * 32;
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ds = 0; ds < 8; ds++) {
      s = T::mfma32(ad.rows(Qb, sub, ds), kf[ds], s);
      dp = T::mfma32(ad.rows(Ob, sub, ds), vf[ds], dp);
    }
    f32x4 l4[4], d4[4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      l4[g] = *(const f32x4*)(Lb + sub * 32 + 8 * g + 4 * h);
      d4[g] = *(const f32x4*)(Db + sub * 32 + 8 * g + 4 * h);
    }
    if (EDGE) {  // a hidden score is -inf: probability 0, or NaN against a row with every key hidden
      const int key = wk0 + n;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const int qq = s0 + 8 * (i >> 2) + 4 * h + (i & 3);
        bool hide = (qq >= t_q) | !live;
        if (CAUSAL) hide |= qq < key;
        s[i] = hide ? neg_inf() : s[i];
      }
    }
#pragma unroll
    for (int i = 0; i < 16; i++) s[i] = fast_exp2(fmaf(s[i], c2, -l4[i >> 2][i & 3]));
#pragma unroll
    for (int i = 0; i < 16; i++) dp[i] = s[i] * fmaf(dp[i], scale, -d4[i >> 2][i & 3]);
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const u16x8 pb = pack8<T>(s, 8 * c), gb = pack8<T>(dp, 8 * c);
#pragma unroll
      for (int dt = 0; dt < 4; dt++) {
        gv[dt] = T::mfma32(ad.transposed(Ob, sub * 32 + 16 * c, dt), pb, gv[dt]);
        gk[dt] = T::mfma32(ad.transposed(Qb, sub * 32 + 16 * c, dt), gb, gk[dt]);
      }
    }
  }
  // per step: the S/dP MFMAs with their 16 row reads and the 8 statistics reads (4 ahead), the
  // softmax, then the dV/dK MFMAs with their 32 transposing reads (4 ahead)
#pragma unroll
  for (int sub = 0; sub < 2; sub++) {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int q = 0; q < 10; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 200, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int q = 0; q < 14; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
}

template <typename T, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 1) void sdpa_bwd_kv_dma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                              const u16* __restrict__ v, const u16* __restrict__ dout,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ delta,
                                                              const u16* __restrict__ mask, u16* __restrict__ dk,
                                                              u16* __restrict__ dv, int64_t batch, int t_q, int t_k,
                                                              float scale) {
  constexpr int D = 128, ROWS = 128;
  __shared__ __attribute__((aligned(1024))) u16 Q0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 Q1[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 O0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 O1[TILE * D];
  __shared__ __attribute__((aligned(16))) float L0[TILE], L1[TILE], D0[TILE], D1[TILE];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  int64_t b, kb;  // causal: the first keys are seen by the most queries
  head_and_block(batch, (t_k + ROWS - 1) / ROWS, b, kb);
  const int k0 = (int)kb * ROWS, wk0 = k0 + wave * 32;
  const Rows krows(k + b * (int64_t)t_k * D, t_k, D), vrows(v + b * (int64_t)t_k * D, t_k, D);
  const DmaTile128 qd(q + b * (int64_t)t_q * D, t_q, wave, lane), od(dout + b * (int64_t)t_q * D, t_q, wave, lane);
  const SwzReads128 ad(lane);
  const float c2 = scale * LOG2E;

  u16x8 kf[8], vf[8];
  f32x16 gk[4], gv[4];
  const int key = wk0 + n;
#pragma unroll
  for (int ds = 0; ds < 8; ds++) {
    kf[ds] = krows.load8(key * D + ds * 16 + 8 * h);
    vf[ds] = vrows.load8(key * D + ds * 16 + 8 * h);
  }
  bool live = key < t_k;
  if (MASK) live = live & (T::unpack(mask[b * (int64_t)t_k + (key < t_k ? key : t_k - 1)]) != 0.f);
#pragma unroll
  for (int dt = 0; dt < 4; dt++) {
    gk[dt] = zero16();
    gv[dt] = zero16();
  }
  const int qstart = CAUSAL ? k0 : 0;  // a causal key is seen by queries at or after it
  const int ntiles = qstart < t_q ? (t_q - qstart + TILE - 1) / TILE : 0;

  // a tile's statistics (lse * log2 e and delta * scale of its queries), by the first wave: loaded
  // into registers when the tile's copy starts and stored into LDS only after the tile before it
  // is computed. Loads retire in order, so using them sooner would wait for the whole copy first.
  float next_l = 0.f, next_d = 0.f;
  auto stats_load = [&](int r0) __attribute__((always_inline)) {
    if (threadIdx.x < TILE) {
      const int qq = r0 + (int)threadIdx.x;
      next_l = qq < t_q ? lse[b * (int64_t)t_q + qq] : 0.f;
      next_d = qq < t_q ? delta[b * (int64_t)t_q + qq] : 0.f;
    }
  };
  auto stats_store = [&](float* L, float* Dl) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);  // keeps the scaling (the loads' first use) below the compute
    if (threadIdx.x < TILE) {
      L[threadIdx.x] = next_l * LOG2E;
      Dl[threadIdx.x] = next_d * scale;
    }
  };
  // tile it from (Qc, Oc, Lc, Dc) while tile it + 1 is copied into the idle buffers (every wave
  // left them at the last barrier), then the wait for the copy and the barrier
  auto step = [&](auto edge, int it, const u16* Qc, const u16* Oc, const float* Lc, const float* Dc, u16* Qn, u16* On,
                  float* Ln, float* Dn) __attribute__((always_inline)) {
    const int r0 = qstart + it * TILE;
    qd.copy(Qn, r0 + TILE, wave);
    od.copy(On, r0 + TILE, wave);
    stats_load(r0 + TILE);
    kv_tile128<T, CAUSAL, MASK, decltype(edge)::value>(Qc, Oc, Lc, Dc, ad, r0, wk0, t_q, c2, scale, live, kf, vf, gk, gv);
    stats_store(Ln, Dn);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    __syncthreads();
  };
  // tiles [from, to) with one body, from even: tile it is in buffer it % 2
  auto run = [&](auto edge, int from, int to) __attribute__((always_inline)) {
    int it = from;
    for (; it + 1 < to; it += 2) {
      step(edge, it, Q0, O0, L0, D0, Q1, O1, L1, D1);
      step(edge, it + 1, Q1, O1, L1, D1, Q0, O0, L0, D0);
    }
    if (it < to) step(edge, it, Q0, O0, L0, D0, Q1, O1, L1, D1);
  };
  if (ntiles > 0) {
    qd.copy(Q0, qstart, wave);
    od.copy(O0, qstart, wave);
    stats_load(qstart);
    stats_store(L0, D0);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    __syncthreads();
  }
  constexpr std::true_type masked{};
  constexpr std::false_type open{};
  if (MASK || ntiles <= 2) {
    run(masked, 0, ntiles);
  } else {
    const int lead = CAUSAL ? 2 : 0, end = t_q % TILE ? ntiles - 1 : ntiles;
    if (lead) run(masked, 0, lead);
    run(open, lead, end);
    if (end < ntiles) {
      if (end & 1) step(masked, end, Q1, O1, L1, D1, Q0, O0, L0, D0);
      else step(masked, end, Q0, O0, L0, D0, Q1, O1, L1, D1);
    }
  }
  store_transposed<T, D>(dk + b * (int64_t)t_k * D, gk, key, t_k, 1.f);
  store_transposed<T, D>(dv + b * (int64_t)t_k * D, gv, key, t_k, 1.f);
}

// ---- the dS hand-off between the dK/dV pass and the dQ pass (D = 128) --------------------------
// The dK/dV pass computes dS = P (dP - delta) scale for every (query, key) pair it visits; the dQ
// pass needs exactly those values (dQ = dS K). Handing them over in memory (2 bytes a pair, as the
// 16-bit operand both products take) replaces the dQ pass's recomputation of S and dP, two of its
// three products and its softmax. Layout, per head: for each 128-key block kb, the 64-query tiles
// the dK/dV pass walks for it (under causality tiles 2 kb onwards, else every tile) as units of
// DS_UNIT bytes, kb after kb; a unit is 16 blocks of 1 KB ordered [wave w][half sub][chunk c], and
// lane L = 32 H + N of a block holds the 8 values of key 32 w + N that the pass packed as the B
// operand of its dK product: queries 16 c + 4 H + {0..3} and 16 c + 8 + 4 H + {0..3} of the half.
constexpr int DS_UNIT = 16384;

struct DsLayout {
  int nqt, nkb;  // 64-query tiles, 128-key blocks per head
  bool causal;
  static __host__ __device__ DsLayout of(int64_t t_q, int64_t t_k, bool causal) {
    return DsLayout{(int)((t_q + TILE - 1) / TILE), (int)((t_k + 127) / 128), causal};
  }
  __host__ __device__ int first_tile(int kb) const { return causal ? 2 * kb : 0; }
  __host__ __device__ int tiles(int kb) const { return nqt - first_tile(kb); }  // units of block kb
  __host__ __device__ int64_t first_unit(int kb) const {
    return causal ? (int64_t)kb * nqt - (int64_t)kb * (kb - 1) : (int64_t)kb * nqt;
  }
  __host__ __device__ int64_t units_per_head() const { return first_unit(nkb); }
};

// ---- dK/dV pass at D = 128 without a key mask: two waves per SIMD -------------------------------
// A workgroup owns 128 keys and is 8 waves: wave w takes keys 32 (w % 4) .. + 31 and queries
// 32 (w / 4) .. + 31 of every 64-query tile, and computes all four products of that 32 x 32
// piece: S = Q K^T and dP = dO V^T (two independent chains over the head dim), P and
// dS = P (dP - delta) scale, then dV^T += dO^T P and dK^T += Q^T dS (transposing reads). The
// block's K and V rows sit in LDS (64 KiB, read as the B operands of S and dP) rather than in
// registers, so a wave fits in 256 registers and two share a SIMD: one's softmax and LDS reads run
// under the other's MFMAs. Each wave reads its operands one 16-deep step ahead. Q and dO tiles
// are double-buffered by DMA, one barrier per tile; the two waves of a key group add their
// partial dK and dV at the end (through LDS, the second query half's onto the first's, in that
// order, so two runs give the same bits). Causal tiles after the first two (which hold the
// block's diagonal) need no mask; rows past t_q arrive as zeros with zero statistics, so P = 1
// there but dS = dO = 0 and they add nothing. Without a key mask no tile but the two diagonal
// ones is masked; masked calls keep sdpa_bwd_kv_dma.
// Measured on the MI355X at 128 heads x 4096 rows, causal, with the dS hand-off (the C4 step),
// alternating builds on one box: 1.189-1.243 ms against 1.257-1.320 for the single-wave pass it
// replaced (K/V in registers, 236 VGPRs + 220 AGPRs, one wave per SIMD, the softmax
// software-pipelined against the next half's products); the same 8-wave pass reading its operands
// in the step rather than one step ahead ran 1.277 against 1.270.
//
// With STORE_DS the pass also hands dS to the dQ pass (sdpa_dq_ds): each 16-query chunk's dS,
// packed as the B operand of its dK product, goes out as it is, one 16-byte store per lane, into
// the layout DsLayout describes (the key group is the block's "wave", the query half its "half").
// The stores go through a buffer resource per tile whose size is zero for the tile past the
// end, so that one is dropped without a branch.
constexpr int KV_WAVES = 8;

template <typename T, bool CAUSAL, bool STORE_DS>
__global__ __launch_bounds__(64 * KV_WAVES, 1) void sdpa_bwd_kv_dual(
    const u16* __restrict__ q, const u16* __restrict__ k, const u16* __restrict__ v, const u16* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, u16* __restrict__ dk, u16* __restrict__ dv,
    u16* __restrict__ dsout, int64_t batch, int t_q, int t_k, float scale) {
  constexpr int D = 128, ROWS = 128;
  // The streamed tiles come first, in the low 64 KiB, where every read's LDS address is a lane
  // offset plus the 16-bit immediate; K and V (the block's rows as two swizzled 64-row tiles
  // each) follow, read at a lane offset that includes their base, V 32 KiB after K.
  __shared__ __attribute__((aligned(1024))) u16 Q0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 Q1[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 O0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 O1[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 Ks[ROWS * D];
  __shared__ __attribute__((aligned(1024))) u16 Vs[ROWS * D];
  __shared__ __attribute__((aligned(16))) float L0[TILE], L1[TILE], D0[TILE], D1[TILE];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int kg = wave & 3, hq = wave >> 2;  // key group, query half
  int64_t b, kb;  // causal: the first keys are seen by the most queries
  head_and_block(batch, (t_k + ROWS - 1) / ROWS, b, kb);
  const int k0 = (int)kb * ROWS, wk0 = k0 + kg * 32, key = wk0 + n;
  const DmaTile128x8 kd(k + b * (int64_t)t_k * D, t_k, wave, lane), vd(v + b * (int64_t)t_k * D, t_k, wave, lane);
  const DmaTile128x8 qd(q + b * (int64_t)t_q * D, t_q, wave, lane), od(dout + b * (int64_t)t_q * D, t_q, wave, lane);
  const float c2 = scale * LOG2E;
  // per-lane byte offsets of every LDS read, the wave's rows folded in, so each read is one of
  // these plus a compile-time offset (the arrays' own): rk by 16-deep step ds into Ks / Vs (this
  // wave's 32 keys), rq by ds into a Q / dO tile (its 32 queries), rt by (dims 32 dt, half jj)
  // for the transposing reads of its queries' first 16-query chunk (the second is 4 KiB on)
  int rk[8], rq[8], rt[4][2];
  {
    const SwzReads128 ad(lane);
#pragma unroll
    for (int ds = 0; ds < 8; ds++) {
      rk[ds] = ad.row[ds] + kg * 32 * 256;  // rows 32 kg + n of the two 64-row tiles, 16 KiB apart
      rq[ds] = ad.row[ds] + hq * 32 * 256;
    }
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int jj = 0; jj < 2; jj++) rt[dt][jj] = ad.tr[dt][jj] + hq * 32 * 256;
  }
  auto rows_at = [](const u16* base, int off) __attribute__((always_inline)) {
    return *(const u16x8*)((const char*)base + off);
  };
  auto transposed_at = [&](const u16* tile, int c, int dt) __attribute__((always_inline)) {
    const char* p = (const char*)tile + c * 16 * 256;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + rt[dt][0]));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + rt[dt][1]));
    return __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16 gk[4], gv[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++) {
    gk[dt] = zero16();
    gv[dt] = zero16();
  }
  const int qstart = CAUSAL ? k0 : 0;  // a causal key is seen by queries at or after it
  const int ntiles = qstart < t_q ? (t_q - qstart + TILE - 1) / TILE : 0;

  const __amdgpu_buffer_rsrc_t lrs = __builtin_amdgcn_make_buffer_rsrc((void*)(lse + b * (int64_t)t_q), (short)0, t_q * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t drs = __builtin_amdgcn_make_buffer_rsrc((void*)(delta + b * (int64_t)t_q), (short)0, t_q * 4, 0x00020000);
  float next_l = 0.f, next_d = 0.f;
  auto stats_load = [&](int r0) __attribute__((always_inline)) {
    next_l = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(lrs, (r0 + lane) * 4, 0, 0));
    next_d = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(drs, (r0 + lane) * 4, 0, 0));
  };
  auto stats_store = [&](float* L, float* Dl) __attribute__((always_inline)) {
    L[lane] = next_l * LOG2E;
    Dl[lane] = next_d * scale;
  };
  const DsLayout lay = DsLayout::of(t_q, t_k, CAUSAL);
  char* const dsk = STORE_DS ? (char*)dsout + ((int64_t)b * lay.units_per_head() + lay.first_unit((int)kb)) * DS_UNIT : nullptr;
  const int ds_voff = kg * 4096 + hq * 2048 + lane * 16;

  // one tile of this wave's 32 queries (half hq of the tile at r0) against its 32 keys
  auto tile = [&](auto edge, int t, const u16* Qc, const u16* Oc, const float* Lc, const float* Dc) __attribute__((always_inline)) {
    constexpr bool EDGE = decltype(edge)::value;
    const int r0 = qstart + t * TILE;
    // the K and V rows are the same every tile: kept from hoisting their reads out of the tile
    // loop, which would hold them in 64 registers (what this pass moves to LDS)
    asm volatile("" ::: "memory");
    f32x16 s = zero16(), dp = zero16();
    // S = Q K^T and dP = dO V^T, 16-deep steps over the head dim, two chains, each step's four
    // operands read one step ahead (deeper, they would not fit two waves' registers)
    u16x8 xa[2][4];
    auto xread = [&](int ds, u16x8* o) __attribute__((always_inline)) {
      o[0] = rows_at(Qc, rq[ds]); o[1] = rows_at(Ks, rk[ds]); o[2] = rows_at(Oc, rq[ds]); o[3] = rows_at(Vs, rk[ds]);
    };
    xread(0, xa[0]);
#pragma unroll
    for (int ds = 0; ds < 8; ds++) {
      if (ds + 1 < 8) xread(ds + 1, xa[(ds + 1) & 1]);
      s = T::mfma32(xa[ds & 1][0], xa[ds & 1][1], s);
      dp = T::mfma32(xa[ds & 1][2], xa[ds & 1][3], dp);
      __builtin_amdgcn_sched_barrier(0);
    }
    unsigned pk[8], gk2[8];
    float pv = 0.f, gv2 = 0.f;
    f32x4 l4, d4;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      if ((i & 3) == 0) {
        l4 = *(const f32x4*)(Lc + hq * 32 + 8 * (i >> 2) + 4 * h);
        d4 = *(const f32x4*)(Dc + hq * 32 + 8 * (i >> 2) + 4 * h);
      }
      float p = fast_exp2(fmaf(s[i], c2, -l4[i & 3]));
      if (EDGE) {
        const int qq = r0 + hq * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        bool hide = (qq >= t_q) | (key >= t_k);
        if (CAUSAL) hide |= qq < key;
        p = hide ? 0.f : p;
      }
      const float g = p * fmaf(dp[i], scale, -d4[i & 3]);
      if (i & 1) {
        pk[i >> 1] = T::pack2(pv, p);
        gk2[i >> 1] = T::pack2(gv2, g);
      } else {
        pv = p;
        gv2 = g;
      }
    }
    u16x8 pb[2], gb[2];
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const u32x4 wp = {pk[4 * c], pk[4 * c + 1], pk[4 * c + 2], pk[4 * c + 3]};
      const u32x4 wg = {gk2[4 * c], gk2[4 * c + 1], gk2[4 * c + 2], gk2[4 * c + 3]};
      pb[c] = __builtin_bit_cast(u16x8, wp);
      gb[c] = __builtin_bit_cast(u16x8, wg);
    }
    if (STORE_DS) {
      const __amdgpu_buffer_rsrc_t dsr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(dsk + (int64_t)t * DS_UNIT), (short)0, t < ntiles ? DS_UNIT : 0, 0x00020000);
#pragma unroll
      for (int c = 0; c < 2; c++)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, gb[c]), dsr, ds_voff + c * 1024, 0, AUX_NT);
    }
    // dV^T += dO^T P and dK^T += Q^T dS over the half's two 16-query chunks
    u16x8 ya[2][2];
    auto yread = [&](int j, u16x8* o) __attribute__((always_inline)) {
      o[0] = transposed_at(Oc, j >> 2, j & 3); o[1] = transposed_at(Qc, j >> 2, j & 3);
    };
    yread(0, ya[0]);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      if (j + 1 < 8) yread(j + 1, ya[(j + 1) & 1]);
      const int c = j >> 2, dt = j & 3;
      gv[dt] = T::mfma32(ya[j & 1][0], pb[c], gv[dt]);
      gk[dt] = T::mfma32(ya[j & 1][1], gb[c], gk[dt]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // tile t from (Qc, Oc, Lc, Dc) while tile t + 1 is copied into (Qn, On) and its statistics
  // loaded; then the wait for those copies (all but the newest two operations, this tile's dS
  // stores, which need not be waited for), the statistics into (Ln, Dn), and the barrier
  auto step = [&](auto edge, int t, const u16* Qc, const u16* Oc, const float* Lc, const float* Dc, u16* Qn, u16* On,
                  float* Ln, float* Dn) __attribute__((always_inline)) {
    const int r1 = qstart + (t + 1) * TILE;
    qd.copy(Qn, r1, wave);
    od.copy(On, r1, wave);
    stats_load(r1);
    __builtin_amdgcn_sched_barrier(0);  // the copies and loads issue before this tile's dS stores
    tile(edge, t, Qc, Oc, Lc, Dc);
    __builtin_amdgcn_s_waitcnt(STORE_DS ? wait_vm(2) : WAIT_VMEM);
    stats_store(Ln, Dn);
    __syncthreads();
  };
  if (ntiles > 0) {
    kd.copy(Ks, k0, wave);
    kd.copy(Ks + TILE * D, k0 + TILE, wave);
    vd.copy(Vs, k0, wave);
    vd.copy(Vs + TILE * D, k0 + TILE, wave);
    qd.copy(Q0, qstart, wave);
    od.copy(O0, qstart, wave);
    stats_load(qstart);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    stats_store(L0, D0);
    __syncthreads();
    constexpr std::true_type masked{};
    constexpr std::false_type whole{};
    // the first two tiles of a causal block hold its diagonal
    int t = 0;
    if (CAUSAL) {
      step(masked, 0, Q0, O0, L0, D0, Q1, O1, L1, D1);
      if (ntiles > 1) step(masked, 1, Q1, O1, L1, D1, Q0, O0, L0, D0);
      t = 2;
    }
    for (; t + 1 < ntiles; t += 2) {
      step(whole, t, Q0, O0, L0, D0, Q1, O1, L1, D1);
      step(whole, t + 1, Q1, O1, L1, D1, Q0, O0, L0, D0);
    }
    if (t < ntiles) step(whole, t, Q0, O0, L0, D0, Q1, O1, L1, D1);
  }
  __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
  __syncthreads();  // every wave is done with every buffer
  // the second query half's partials to LDS, in its accumulators' own lane order, 16 KiB per
  // matrix: key group 0 in Ks, 1 in Vs, 2 in Q0 / Q1, 3 in O0 / O1
  char* const part_k = kg == 0 ? (char*)Ks : kg == 1 ? (char*)Vs : kg == 2 ? (char*)Q0 : (char*)O0;
  char* const part_v = kg == 0 ? (char*)Ks + 16384 : kg == 1 ? (char*)Vs + 16384 : kg == 2 ? (char*)Q1 : (char*)O1;
  if (hq == 1) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        *(f32x4*)(part_k + ((dt * 4 + e) * 64 + lane) * 16) = f32x4{gk[dt][4 * e], gk[dt][4 * e + 1], gk[dt][4 * e + 2], gk[dt][4 * e + 3]};
        *(f32x4*)(part_v + ((dt * 4 + e) * 64 + lane) * 16) = f32x4{gv[dt][4 * e], gv[dt][4 * e + 1], gv[dt][4 * e + 2], gv[dt][4 * e + 3]};
      }
  }
  __syncthreads();
  if (hq == 0) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const f32x4 pk4 = *(const f32x4*)(part_k + ((dt * 4 + e) * 64 + lane) * 16);
        const f32x4 pv4 = *(const f32x4*)(part_v + ((dt * 4 + e) * 64 + lane) * 16);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          gk[dt][4 * e + j] = gk[dt][4 * e + j] + pk4[j];
          gv[dt][4 * e + j] = gv[dt][4 * e + j] + pv4[j];
        }
      }
    // staged through this key group's dK partial area (8704 of its 16384 bytes), which only this
    // wave reads from now on (LDS runs a wave's operations in order)
    u16* stage = (u16*)part_k;
    store_staged<T, 128>(dk + b * (int64_t)t_k * D, gk, wk0, t_k, 1.f, stage);
    store_staged<T, 128>(dv + b * (int64_t)t_k * D, gv, wk0, t_k, 1.f, stage);
  }
}

// ---- dQ pass from the handed-over dS (D = 128) --------------------------------------------------
// dQ^T += K^T dS^T with the resident queries on the N side, as sdpa_bwd_q_dma, but dS comes from
// the dK/dV pass's hand-off instead of being recomputed: a third of that pass's products, no
// softmax, and 2 bytes of dS streamed per (query, key) pair, so the pass is bound by HBM. Per
// 64-key step a workgroup copies the K tile (swizzled, as in the other passes) and the dS of its
// 128 queries (16 blocks of 1 KB: tile e = wave / 2, kv-wave 2 hh + wave % 2, [half][chunk]) into
// LDS by DMA. A block's lanes hold (key, 8 queries) and the B operand needs (query, 8 keys):
// ds_read_b64_tr_b16 turns the one into the other when lane a of each 16-lane group addresses
// 4 consecutive queries of one key, key 16 kc + 4 h + a / 4 (+ 8 for the operand's second half),
// queries 4 (a % 4) .. + 3 of the group's 16-query chunk, which matches the key order of the
// transposed K operand. The DMA lanes place raw lane 32 H + N of chunk c at slot
// 32 H + 16 (N / 16) + ((N + 8 c + 4 H) mod 16) of its block, so the 32 lanes of each half of a
// read touch 32 distinct 8-byte bank pairs.

// one 64-key step: dQ^T of the wave's 32 queries += K^T dS^T over four 16-key chunks
template <typename T>
__device__ __forceinline__ void dq_step128(const u16* Kb, const u16* Sb, const SwzReads128& ad, const int (&soff)[2],
                                           f32x16 (&acc)[4]) {
#pragma unroll
  for (int kc = 0; kc < 4; kc++) {
    const char* p = (const char*)Sb + (kc >> 1) * 4096 + (kc & 1) * 256;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + soff[0]));
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p + soff[1]));
    const u16x8 g = __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
    for (int dt = 0; dt < 4; dt++) acc[dt] = T::mfma32(ad.transposed(Kb, 16 * kc, dt), g, acc[dt]);
  }
}

template <typename T, bool CAUSAL>
__global__ __launch_bounds__(THREADS, 2) void sdpa_dq_ds(const u16* __restrict__ k, const u16* __restrict__ dsin,
                                                         u16* __restrict__ dq, int64_t batch, int t_q, int t_k) {
  constexpr int D = 128, ROWS = 128;
  __shared__ __attribute__((aligned(1024))) u16 K0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 K1[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 S0[TILE * D];  // dS of 128 queries x 64 keys
  __shared__ __attribute__((aligned(1024))) u16 S1[TILE * D];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nqb = (t_q + ROWS - 1) / ROWS;
  int64_t b, blk;
  head_and_block<DQ_HEAD_GROUP>(batch, nqb, b, blk);
  // heads in the reverse of the dK/dV pass's order: every XCD starts on a head whose dS that
  // pass wrote last, part of which the Infinity Cache still holds. Measured on the MI355X at 128
  // heads x 4096 rows, causal, alternating builds on one box: 0.4932 against 0.5011-0.5015 ms,
  // 0.4735-0.4737 against 0.4760-0.4763 on another.
  b = batch - 1 - b;
  const int qb = (int)(nqb - 1 - blk);  // causal: the longest rows go first
  const int q0 = qb * ROWS;
  const DsLayout lay = DsLayout::of(t_q, t_k, CAUSAL);
  const char* const dsh = (const char*)dsin + b * lay.units_per_head() * DS_UNIT;
  const DmaTile128 kd(k + b * (int64_t)t_k * D, t_k, wave, lane);
  const SwzReads128 ad(lane);

  // copies: DMA lane s of chunk c's block loads raw lane src of the block (see above)
  int src[2];
#pragma unroll
  for (int c = 0; c < 2; c++) {
    const int s = lane, hs = s >> 5;
    const int raw = 32 * hs + 16 * ((s >> 4) & 1) + (((s & 15) - 8 * c - 4 * hs) & 15);
    src[c] = raw * 16 + c * 1024 + (wave & 1) * 4096;
  }
  // B operand reads: the wave's tile e and half, the lane's chunk c = (lane / 16) % 2, key offset
  // 0 or 8; a key chunk kc adds (kc / 2) * 4096 + (kc % 2) * 256
  int soff[2];
  {
    const int g = lane >> 4, h = lane >> 5, a = lane & 15, c = g & 1, hp = a & 1, x = (a >> 1) & 1;
#pragma unroll
    for (int sec = 0; sec < 2; sec++)
      soff[sec] = (8 * (wave >> 1) + 2 * (wave & 1) + c) * 1024 + 512 * hp + 8 * x +
                  ((8 * sec + 4 * h + (a >> 2) + 8 * c + 4 * hp) & 15) * 16;
  }
  // step s covers keys [64 s, 64 s + 64): block kb = s / 2, its half hh = s % 2. A unit that does
  // not exist (past the key blocks, or a query tile the dK/dV pass did not walk) copies nothing.
  auto copy_ds = [&](u16* S, int s) __attribute__((always_inline)) {
    const int kb = s >> 1, hh = s & 1;
    const int rel = 2 * qb + (wave >> 1) - lay.first_tile(kb);
    const bool ok = kb < lay.nkb && rel >= 0 && rel < lay.tiles(kb);
    const char* base = ok ? dsh + (lay.first_unit(kb) + rel) * DS_UNIT + hh * 8192 : dsh;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, ok ? 8192 : 0, 0x00020000);
#pragma unroll
    for (int blk4 = 0; blk4 < 4; blk4++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)((char*)S + (wave * 4 + blk4) * 1024), 16,
                                               src[blk4 & 1] + (blk4 >> 1) * 2048, 0, 0, AUX_NT);
  };

  f32x16 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++) acc[dt] = zero16();
  const int nsteps = 2 * (CAUSAL ? qb + 1 : lay.nkb);
  auto step = [&](int s, const u16* Kc, const u16* Sc, u16* Kn, u16* Sn) __attribute__((always_inline)) {
    kd.copy(Kn, (s + 1) * TILE, wave);
    copy_ds(Sn, s + 1);
    dq_step128<T>(Kc, Sc, ad, soff, acc);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    __syncthreads();
  };
  kd.copy(K0, 0, wave);
  copy_ds(S0, 0);
  __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
  __syncthreads();
  for (int s = 0; s < nsteps; s += 2) {  // nsteps is even
    step(s, K0, S0, K1, S1);
    step(s + 1, K1, S1, K0, S0);
  }
  u16* stage = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? S0 : S1;  // free after the last barrier
  store_staged<T, 128>(dq + b * (int64_t)t_q * D, acc, q0 + wave * 32, t_q, 1.f, stage);
}

// The unmasked D = 128 dK/dV pass (dk, dv out; with STORE_DS the dS hand-off into ds).
template <typename T, bool CAUSAL, bool STORE_DS>
int launch_kv128(const SdpaArgs& a, u16* dk, u16* dv, u16* ds) {
  const int64_t blocks = a.batch * ((a.t_k + 127) / 128);
  if (blocks > 0x7fffffff) return fail(LIMN_HIP_EUNSUPPORTED, "sdpa: %lld workgroups exceed one launch", (long long)blocks);
  hipLaunchKernelGGL((sdpa_bwd_kv_dual<T, CAUSAL, STORE_DS>), dim3((unsigned)blocks), dim3(64 * KV_WAVES), 0, a.stream,
                     (const u16*)a.q, (const u16*)a.k, (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse,
                     (const float*)a.delta, dk, dv, ds, a.batch, (int)a.t_q, (int)a.t_k, (float)a.scale);
  return check_hip(hipGetLastError(), "launching the dK/dV pass");
}

// The dK/dV pass with the dS hand-off, then the dQ pass reading it: both backward CUSTOM kernels
// in two launches, `ws` holding batch * DsLayout::units_per_head() * DS_UNIT bytes; `passes`
// (LIMN_HIP_BWD_* bits) may pick one of the two.
template <typename T, bool CAUSAL>
int launch_bwd_ds(const SdpaArgs& a, void* ws, int passes) {
  const int64_t nkb = (a.t_k + 127) / 128, nqb = (a.t_q + 127) / 128;
  if (a.batch * nkb > 0x7fffffff || a.batch * nqb > 0x7fffffff)
    return fail(LIMN_HIP_EUNSUPPORTED, "sdpa_bwd: %lld heads exceed one launch", (long long)a.batch);
  if (passes & LIMN_HIP_BWD_KV_PASS) {
    const int rc = launch_kv128<T, CAUSAL, true>(a, (u16*)a.out1, (u16*)a.out2, (u16*)ws);
    if (rc != LIMN_HIP_OK) return rc;
  }
  if (!(passes & LIMN_HIP_BWD_Q_PASS)) return LIMN_HIP_OK;
  hipLaunchKernelGGL((sdpa_dq_ds<T, CAUSAL>), dim3((unsigned)(a.batch * nqb)), dim3(THREADS), 0, a.stream, (const u16*)a.k,
                     (const u16*)ws, (u16*)a.out0, a.batch, (int)a.t_q, (int)a.t_k);
  return check_hip(hipGetLastError(), "launching the dQ pass");
}

// ---- forward at D = 128: streamed K and V tiles copied straight into LDS ------------------------
// The same swizzled tiles and LDS DMA as the dK/dV pass above: K is read as row operands of
// S^T = K Q^T, V through the transposing reads of O^T += V^T P^T. Tiles that need masking (a
// causal block's two diagonal tiles, a last tile past t_k, every tile under a key mask) run
// their own instance of the tile body.

// Each wave keeps 32 queries resident and walks 64-key tiles: S^T for both 32-key halves, one
// online softmax step for the 64 keys (the reference point moves only when the tile's max passes
// it by `lift`), then the V^T P^T products. One step per 64 keys rather than per 32 halves the
// serial max / exchange / test chain per key; measured 0.566 ms against 0.587 for the forward at
// 128 heads x 4096 rows, causal (the results differ in rounding: P's reference point moves less
// often).

// The online-softmax update for one 64-key tile of S^T (both 32-key halves, masked when EDGE):
// the tile's max, and when it passes the reference point by more than `lift`, the new reference
// with l and the accumulators rescaled to it
template <bool CAUSAL, bool MASK, bool EDGE>
__device__ __forceinline__ void fwd_max128(f32x16 (&s)[2], int k0, int row, int t_k, float c2, float lift, uint64_t live,
                                           f32x16 (&acc)[4], float& m, float& l) {
  const int lane = threadIdx.x & 63, h = lane >> 5;
  if (EDGE) {
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      const unsigned mb = (unsigned)(live >> (sub * 32 + 4 * h));
#pragma unroll
      for (int i = 0; i < 16; i++) s[sub][i] = hidden<CAUSAL, MASK>(k0, sub, i, h, t_k, row, mb) ? neg_inf() : s[sub][i];
    }
  }
  float mx = neg_inf();
#pragma unroll
  for (int sub = 0; sub < 2; sub++)
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, s[sub][i]);
  mx = pair_max(mx);
  if (__any(mx > m + lift)) {
    const float mnew = fmaxf(m, mx);
    const float alpha = mnew == neg_inf() ? 1.f : fast_exp2((m - mnew) * c2);
    l *= alpha;
#pragma unroll
    for (int dt = 0; dt < 4; dt++) acc[dt] *= alpha;
    m = mnew;
  }
}

// S^T of one 64-key tile against the wave's 32 resident queries, both 32-key halves
template <typename T>
__device__ __forceinline__ void fwd_scores128(const u16* Kb, const SwzReads128& ad, const u16x8 (&qf)[8], f32x16 (&s)[2]) {
  s[0] = zero16();
  s[1] = zero16();
#pragma unroll
  for (int ds = 0; ds < 8; ds++)
#pragma unroll
    for (int sub = 0; sub < 2; sub++) s[sub] = T::mfma32(ad.rows(Kb, sub, ds), qf[ds], s[sub]);
}

// One pipelined step of the forward: the probabilities of tile `it` (its S^T in `s`, the reference
// point already moved for it) and the V^T P^T products from Vc, while the S^T products of tile
// it + 1 (from Kn) run on the matrix cores; then tile it + 1's online-softmax update. The
// exponentials of one tile and the scores of the next are independent, so the wave issues VALU
// work while its own MFMAs execute instead of waiting on them. Same operations in the same order
// per element as one tile at a time, so the same bits. Measured on the MI355X at 128 heads x 4096
// rows, causal, alternating builds on one box: 0.544-0.550 ms against 0.560-0.566 for one tile at
// a time; pinning the interleave (one LDS read and six VALU instructions per MFMA, by
// sched_group_barrier) ran 0.552-0.558, the compiler's own order is kept.
template <typename T, bool CAUSAL, bool MASK, bool EDGE_NEXT, bool HAS_NEXT>
__device__ __forceinline__ void fwd_pipe128(const u16* Kn, const u16* Vc, const SwzReads128& ad, int kn0, int row, int t_k,
                                            float c2, float lift, uint64_t live_next, const u16x8 (&qf)[8],
                                            f32x16 (&acc)[4], f32x16 (&s)[2], float& m, float& l) {
  f32x16 sn[2];
  if (HAS_NEXT) fwd_scores128<T>(Kn, ad, qf, sn);
  const float base = m == neg_inf() ? 0.f : m * c2;
  float rs = 0.f;
#pragma unroll
  for (int sub = 0; sub < 2; sub++)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float p = fast_exp2(fmaf(s[sub][i], c2, -base));
      s[sub][i] = p;
      rs += p;
    }
  l += rs;
#pragma unroll
  for (int sub = 0; sub < 2; sub++)
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const u16x8 pb = pack8<T>(s[sub], 8 * c);
#pragma unroll
      for (int dt = 0; dt < 4; dt++) acc[dt] = T::mfma32(ad.transposed(Vc, sub * 32 + 16 * c, dt), pb, acc[dt]);
    }
  if (HAS_NEXT) {
    fwd_max128<CAUSAL, MASK, EDGE_NEXT>(sn, kn0, row, t_k, c2, lift, live_next, acc, m, l);
    s[0] = sn[0];
    s[1] = sn[1];
  }
}

template <typename T, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 2) void sdpa_fwd_dma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                           const u16* __restrict__ v, const u16* __restrict__ mask,
                                                           u16* __restrict__ out, float* __restrict__ lse, int64_t batch,
                                                           int t_q, int t_k, float scale) {
  constexpr int D = 128, ROWS = 128;
  __shared__ __attribute__((aligned(1024))) u16 K0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 K1[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 V0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 V1[TILE * D];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + ROWS - 1) / ROWS;
  int64_t b, blk;
  head_and_block(batch, nqb, b, blk);
  const int64_t qb = nqb - 1 - blk;  // causal: the longest rows go first
  const int q0 = (int)qb * ROWS, row = q0 + wave * 32 + n;
  const Rows qrows(q + b * (int64_t)t_q * D, t_q, D);
  const DmaTile128 kd(k + b * (int64_t)t_k * D, t_k, wave, lane), vd(v + b * (int64_t)t_k * D, t_k, wave, lane);
  const SwzReads128 ad(lane);
  const MaskRow mrow(MASK ? mask + b * (int64_t)t_k : nullptr, t_k);
  const float c2 = scale * LOG2E, lift = RESCALE_LOG2 / c2;  // scale > 0 (the C ABI routes others away)

  u16x8 qf[8];
  f32x16 acc[4], s[2];
  float m = neg_inf(), l = 0.f;
#pragma unroll
  for (int ds = 0; ds < 8; ds++) qf[ds] = qrows.load8(row * D + ds * 16 + 8 * h);
#pragma unroll
  for (int dt = 0; dt < 4; dt++) acc[dt] = zero16();

  const int kend = CAUSAL ? (q0 + ROWS < t_k ? q0 + ROWS : t_k) : t_k;
  const int ntiles = (kend + TILE - 1) / TILE;
  // unmasked: every key of the tile exists and, under causality, precedes the block's first row
  int open = MASK ? 0 : t_k / TILE;
  if (CAUSAL && q0 / TILE < open) open = q0 / TILE;
  if (open > ntiles) open = ntiles;
  auto live_of = [&](int k0) __attribute__((always_inline)) { return MASK ? live_keys<T>(mrow.load(k0 + lane)) : ~0ull; };
  // Tile it's probabilities and V^T P^T from buffer it % 2, tile it + 1's scores from K buffer
  // (it + 1) % 2, while K of tile it + 2 is copied into K buffer it % 2 and V of tile it + 1
  // into V buffer (it + 1) % 2 (both last read before the previous barrier); then the wait for
  // the copies and the barrier
  auto step = [&](auto edge_next, int it, const u16* Kn, const u16* Vc, u16* Kf, u16* Vf) __attribute__((always_inline)) {
    const int kn0 = (it + 1) * TILE;
    kd.copy(Kf, kn0 + TILE, wave);
    vd.copy(Vf, kn0, wave);
    fwd_pipe128<T, CAUSAL, MASK, decltype(edge_next)::value, true>(Kn, Vc, ad, kn0, row, t_k, c2, lift, live_of(kn0), qf,
                                                                    acc, s, m, l);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    __syncthreads();
  };
  // steps [from, to) whose next tiles share one masking body
  auto run = [&](auto edge_next, int from, int to) __attribute__((always_inline)) {
    int it = from;
    if ((it & 1) && it < to) {
      step(edge_next, it, K0, V1, K1, V0);
      it++;
    }
    for (; it + 1 < to; it += 2) {
      step(edge_next, it, K1, V0, K0, V1);
      step(edge_next, it + 1, K0, V1, K1, V0);
    }
    if (it < to) step(edge_next, it, K1, V0, K0, V1);
  };
  if (ntiles > 0) {
    kd.copy(K0, 0, wave);
    vd.copy(V0, 0, wave);
    kd.copy(K1, TILE, wave);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    __syncthreads();
    fwd_scores128<T>(K0, ad, qf, s);
    if (open > 0)
      fwd_max128<CAUSAL, MASK, false>(s, 0, row, t_k, c2, lift, live_of(0), acc, m, l);
    else
      fwd_max128<CAUSAL, MASK, true>(s, 0, row, t_k, c2, lift, live_of(0), acc, m, l);
    __syncthreads();  // every wave's reads of K buffer 0 are done before tile 2 is copied there
    // step it's next tile is it + 1: unmasked while it + 1 < open
    const int last = ntiles - 1, split = open - 1 < 0 ? 0 : (open - 1 < last ? open - 1 : last);
    run(std::false_type{}, 0, split);
    run(std::true_type{}, split, last);
    const u16* Vl = (last & 1) ? V1 : V0;
    fwd_pipe128<T, CAUSAL, MASK, true, false>(K0, Vl, ad, 0, row, t_k, c2, lift, 0, qf, acc, s, m, l);
    __syncthreads();  // the tile buffers become staging below
  }
  const float total = pair_sum(l);
  u16* stage = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? V0 : V1;
  store_staged<T, 128>(out + b * (int64_t)t_q * D, acc, q0 + wave * 32, t_q, 1.f / total, stage);
  if (h == 0 && row < t_q) lse[b * (int64_t)t_q + row] = m * scale + logf(total);
}

// ---- dQ pass at D = 128: streamed K and V tiles copied straight into LDS ------------------------
// K serves as the row operand of S = Q K^T (taken as S^T = K Q^T) and through transposing reads
// as the operand of dQ^T += K^T dS^T; V as the row operand of dP^T = V dO^T.

// one 64-key tile against the wave's 32 resident queries: per 32-key half, S^T and dP^T, the
// probabilities from the saved log-sum-exp, dS, then the K^T dS^T products
template <typename T, bool CAUSAL, bool MASK, bool EDGE>
__device__ __forceinline__ void q_tile128(const u16* Kb, const u16* Vb, const SwzReads128& ad, int k0, int row, int t_k,
                                          float c2, float scale, float L2, float Dr, uint64_t live,
                                          const u16x8 (&qf)[8], const u16x8 (&of)[8], f32x16 (&acc)[4]) {
  const int lane = threadIdx.x & 63, h = lane >> 5;
#pragma unroll
  for (int sub = 0; sub < 2; sub++) {
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int ds = 0; ds < 8; ds++) {
      s = T::mfma32(ad.rows(Kb, sub, ds), qf[ds], s);
      dp = T::mfma32(ad.rows(Vb, sub, ds), of[ds], dp);
    }
    if (EDGE) {  // a hidden score is -inf: probability 0, or NaN in a row with every key hidden
      const unsigned mb = (unsigned)(live >> (sub * 32 + 4 * h));
#pragma unroll
      for (int i = 0; i < 16; i++) s[i] = hidden<CAUSAL, MASK>(k0, sub, i, h, t_k, row, mb) ? neg_inf() : s[i];
    }
#pragma unroll
    for (int i = 0; i < 16; i++) s[i] = fast_exp2(fmaf(s[i], c2, -L2));
#pragma unroll
    for (int i = 0; i < 16; i++) s[i] *= fmaf(dp[i], scale, -Dr);
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const u16x8 g = pack8<T>(s, 8 * c);
#pragma unroll
      for (int dt = 0; dt < 4; dt++) acc[dt] = T::mfma32(ad.transposed(Kb, sub * 32 + 16 * c, dt), g, acc[dt]);
    }
  }
  // per half: the S/dP MFMAs with their 16 row reads (4 ahead), the probabilities and dS, then the
  // dQ MFMAs with their 16 transposing reads (4 ahead)
#pragma unroll
  for (int sub = 0; sub < 2; sub++) {
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int q = 0; q < 12; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 200, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int q = 0; q < 6; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
  }
}

template <typename T, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(THREADS, 2) void sdpa_bwd_q_dma(const u16* __restrict__ q, const u16* __restrict__ k,
                                                             const u16* __restrict__ v, const u16* __restrict__ dout,
                                                             const float* __restrict__ lse,
                                                             const float* __restrict__ delta,
                                                             const u16* __restrict__ mask, u16* __restrict__ dq,
                                                             int64_t batch, int t_q, int t_k, float scale) {
  constexpr int D = 128, ROWS = 128;
  __shared__ __attribute__((aligned(1024))) u16 K0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 K1[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 V0[TILE * D];
  __shared__ __attribute__((aligned(1024))) u16 V1[TILE * D];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), h = lane >> 5, n = lane & 31;
  const int64_t nqb = (t_q + ROWS - 1) / ROWS;
  int64_t b, blk;
  head_and_block(batch, nqb, b, blk);
  const int64_t qb = nqb - 1 - blk;  // causal: the longest rows go first
  const int q0 = (int)qb * ROWS, row = q0 + wave * 32 + n;
  const Rows qrows(q + b * (int64_t)t_q * D, t_q, D), orows(dout + b * (int64_t)t_q * D, t_q, D);
  const DmaTile128 kd(k + b * (int64_t)t_k * D, t_k, wave, lane), vd(v + b * (int64_t)t_k * D, t_k, wave, lane);
  const SwzReads128 ad(lane);
  const MaskRow mrow(MASK ? mask + b * (int64_t)t_k : nullptr, t_k);
  const float c2 = scale * LOG2E;

  u16x8 qf[8], of[8];
  f32x16 acc[4];
#pragma unroll
  for (int ds = 0; ds < 8; ds++) {
    qf[ds] = qrows.load8(row * D + ds * 16 + 8 * h);
    of[ds] = orows.load8(row * D + ds * 16 + 8 * h);
  }
  const float L2 = row < t_q ? lse[b * (int64_t)t_q + row] * LOG2E : 0.f;
  const float Dr = row < t_q ? delta[b * (int64_t)t_q + row] * scale : 0.f;  // ds = p (dp scale - delta scale)
#pragma unroll
  for (int dt = 0; dt < 4; dt++) acc[dt] = zero16();

  const int kend = CAUSAL ? (q0 + ROWS < t_k ? q0 + ROWS : t_k) : t_k;
  const int ntiles = (kend + TILE - 1) / TILE;
  auto step = [&](auto edge, int it, const u16* Kc, const u16* Vc, u16* Kn, u16* Vn) __attribute__((always_inline)) {
    const int k0 = it * TILE;
    kd.copy(Kn, k0 + TILE, wave);
    vd.copy(Vn, k0 + TILE, wave);
    const uint64_t live = MASK ? live_keys<T>(mrow.load(k0 + lane)) : ~0ull;
    q_tile128<T, CAUSAL, MASK, decltype(edge)::value>(Kc, Vc, ad, k0, row, t_k, c2, scale, L2, Dr, live, qf, of, acc);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    __syncthreads();
  };
  auto run = [&](auto edge, int from, int to) __attribute__((always_inline)) {
    int it = from;
    if ((it & 1) && it < to) {
      step(edge, it, K1, V1, K0, V0);
      it++;
    }
    for (; it + 1 < to; it += 2) {
      step(edge, it, K0, V0, K1, V1);
      step(edge, it + 1, K1, V1, K0, V0);
    }
    if (it < to) step(edge, it, K0, V0, K1, V1);
  };
  if (ntiles > 0) {
    kd.copy(K0, 0, wave);
    vd.copy(V0, 0, wave);
    __builtin_amdgcn_s_waitcnt(WAIT_VMEM);
    __syncthreads();
  }
  int open = MASK ? 0 : t_k / TILE;
  if (CAUSAL && q0 / TILE < open) open = q0 / TILE;
  if (open > ntiles) open = ntiles;
  run(std::false_type{}, 0, open);
  run(std::true_type{}, open, ntiles);
  u16* stage = wave == 0 ? K0 : wave == 1 ? K1 : wave == 2 ? V0 : V1;  // free after the last barrier
  store_staged<T, 128>(dq + b * (int64_t)t_q * D, acc, q0 + wave * 32, t_q, 1.f, stage);
}

// ---------------------------------------------------------------------------------------------

// Resident 32-row tiles per wave for each pass and head dim. The kernels take NT = 2 (each LDS
// operand read feeds two MFMAs), but one tile per wave with two workgroups per CU (two waves per
// SIMD) hides latency better wherever it fits: the D = 64 passes of the GPT step took 448 / 662
// us per step (dQ / dK dV) at two tiles and 288 / 442 us at one; at D = 128 the dK/dV pass's
// accumulators fill the register file at one tile (its LDS-DMA kernel, one workgroup per CU).
template <int D>
constexpr int tiles_per_wave(SdpaPass) {
  return 1;
}

template <typename T, int D, int NT, bool CAUSAL, bool MASK, SdpaPass PASS>
int launch_nt(const SdpaArgs& a) {
  constexpr SdpaPass pass = PASS;
  const int64_t rows = pass == SDPA_BWD_KV ? a.t_k : a.t_q;
  const int64_t per = 128 * NT;
  // the D = 128 kernels take a block each; the D = 64 ones a unit of paired blocks
  const int64_t per_head = (rows + per - 1) / per;
  const int64_t blocks = a.batch * (D == 128 ? per_head : paired_units<CAUSAL>(per_head));
  if (blocks > 0x7fffffff) return fail(LIMN_HIP_EUNSUPPORTED, "sdpa: %lld workgroups exceed one launch", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(THREADS);
  const float scale = (float)a.scale;
  const u16* mask = (const u16*)a.mask;
  if constexpr (PASS == SDPA_FWD && D == 128) {
    hipLaunchKernelGGL((sdpa_fwd_dma<T, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q, (const u16*)a.k,
                       (const u16*)a.v, mask, (u16*)a.out0, (float*)a.out1, a.batch, (int)a.t_q, (int)a.t_k, scale);
  } else if constexpr (PASS == SDPA_FWD) {
    hipLaunchKernelGGL((sdpa_fwd_mfma<T, D, NT, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                       (const u16*)a.k, (const u16*)a.v, mask, (u16*)a.out0, (float*)a.out1, a.batch, (int)a.t_q, (int)a.t_k,
                       scale);
  } else if constexpr (PASS == SDPA_BWD_Q && D == 128) {
    hipLaunchKernelGGL((sdpa_bwd_q_dma<T, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q, (const u16*)a.k,
                       (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse, (const float*)a.delta, mask,
                       (u16*)a.out0, a.batch, (int)a.t_q, (int)a.t_k, scale);
  } else if constexpr (PASS == SDPA_BWD_Q) {
    hipLaunchKernelGGL((sdpa_bwd_q_mfma<T, D, NT, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                       (const u16*)a.k, (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse, (const float*)a.delta,
                       mask, (u16*)a.out0, a.batch, (int)a.t_q, (int)a.t_k, scale);
  } else if constexpr (D == 128 && !MASK) {
    return launch_kv128<T, CAUSAL, false>(a, (u16*)a.out0, (u16*)a.out1, nullptr);
  } else if constexpr (D == 128) {
    hipLaunchKernelGGL((sdpa_bwd_kv_dma<T, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q, (const u16*)a.k,
                       (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse, (const float*)a.delta, mask,
                       (u16*)a.out0, (u16*)a.out1, a.batch, (int)a.t_q, (int)a.t_k, scale);
  } else {
    hipLaunchKernelGGL((sdpa_bwd_kv_mfma<T, D, NT, CAUSAL, MASK>), grid, block, 0, a.stream, (const u16*)a.q,
                       (const u16*)a.k, (const u16*)a.v, (const u16*)a.dout, (const float*)a.lse, (const float*)a.delta,
                       mask, (u16*)a.out0, (u16*)a.out1, a.batch, (int)a.t_q, (int)a.t_k, scale);
  }
  return check_hip(hipGetLastError(), "launching an sdpa kernel");
}

template <typename T, int D, SdpaPass PASS>
int launch_flags(const SdpaArgs& a) {
  constexpr int NT = tiles_per_wave<D>(PASS);
  const bool masked = a.mask != nullptr;
  if (a.causal) return masked ? launch_nt<T, D, NT, true, true, PASS>(a) : launch_nt<T, D, NT, true, false, PASS>(a);
  return masked ? launch_nt<T, D, NT, false, true, PASS>(a) : launch_nt<T, D, NT, false, false, PASS>(a);
}

// One pass of the MFMA family at the call's dtype, head dim, causality and masking.
template <SdpaPass PASS>
int launch_pass(const SdpaArgs& a) {
  if (a.dtype == LIMN_HIP_BFLOAT16) return a.hd == 64 ? launch_flags<BF16, 64, PASS>(a) : launch_flags<BF16, 128, PASS>(a);
  return a.hd == 64 ? launch_flags<F16, 64, PASS>(a) : launch_flags<F16, 128, PASS>(a);
}

}  // namespace
}  // namespace limn
