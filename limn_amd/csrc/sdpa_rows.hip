// General-width fused attention: every float dtype (f64, f32, f16, bf16), any head dims up to
// 256, rectangular keys, causal and key masks.
//
// A workgroup is 256 threads owning 64 resident rows (query rows for the forward and dQ pass,
// key rows for the dK/dV pass); each row is held by LANES = 4 neighbouring lanes that split its
// head dims (lane sub-index u holds dims u, u+4, u+8, ...), so a dot product is a per-lane
// partial plus two shuffles. The other operand streams through LDS in tiles of STREAM rows at
// compute width; the 4 lanes of a row read 4 consecutive words and every row reads the same
// streamed row, so reads are conflict-free broadcasts.
//
// With few resident rows per head the workgroups would be too few to fill the GPU and each row's
// walk over the streamed rows one long chain of dependent steps: then (SPLIT = 4, 8 or 16) a row
// is held by SPLIT groups of LANES lanes, group g taking the streamed rows g, g + SPLIT, ... of
// every tile, and the groups' partial results are combined at the end in a fixed butterfly
// (the forward's as (max, total, accumulator) triples rescaled to the common max).
//
// This family carries the widths the MFMA kernels do not (f32 and f64 above all, where the
// reference's tolerances are 1e-5 and 1e-12): it computes in the dtype's compute width with
// natural exp/log, folding streamed rows in ascending order.
//
// Semantics per pass (reference limn/sdpa.py:91-203):
//   forward: online softmax; a key only rescales the running totals when it raises the row max;
//            out = acc / l, lse = m + log(l); a row with every key hidden is NaN with lse -inf.
//   dQ:      p = exp(s*scale - lse); ds = p (dout.v - delta) scale; dq += ds k.
//   dK, dV:  the same p and ds per (query, key); dv += p dout, dk += ds q; hidden keys are 0.

#include "sdpa.h"

namespace limn {
namespace {

constexpr int LANES = 4;                     // lanes per resident row and key group
constexpr int THREADS = 256;                 // per workgroup
// Streamed rows per LDS tile: 32 KiB of each streamed matrix at compute width, from 16 to 128
// rows. Short heads are bound by the staging (a tile's global loads, then two barriers), not by
// the few dot products per row a tile carries: at f32 and 64 dims, 128-row tiles take a 256-key
// causal pass in 2 stages instead of 8. A multiple of every SPLIT, so each lane group folds the
// same keys in the same order whatever the tile.
template <typename C, int MAXD>
constexpr int stream_rows() {
  constexpr int rows = 32768 / (MAXD * (int)sizeof(C));
  return rows > 128 ? 128 : rows < 16 ? 16 : rows;
}
// resident rows per workgroup when each row's streamed rows are split among SPLIT groups of lanes
template <int SPLIT>
constexpr int rows_per_block() { return THREADS / (LANES * SPLIT); }

template <typename C>
__device__ __forceinline__ C exp_c(C x);
template <>
__device__ __forceinline__ float exp_c<float>(float x) { return expf(x); }
template <>
__device__ __forceinline__ double exp_c<double>(double x) { return exp(x); }
template <typename C>
__device__ __forceinline__ C log_c(C x);
template <>
__device__ __forceinline__ float log_c<float>(float x) { return logf(x); }
template <>
__device__ __forceinline__ double log_c<double>(double x) { return log(x); }

// Sum of one value over the LANES lanes of a row (all 4 get the total).
template <typename C>
__device__ __forceinline__ C row_sum(C x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  return x;
}

// LDS row stride of a streamed tile: MAXD + LANES elements. With SPLIT lane groups each group
// reads its own streamed row, lane u of a group dims u, u + 4, ...; at a stride of MAXD (a
// multiple of the 64 banks) every group's row sat on the same four banks and a read was a
// 16-way conflict, at MAXD + 4 words the 16 groups' rows start 4 banks apart.
template <int MAXD>
constexpr int row_stride() { return MAXD + LANES; }

// Stage rows [r0, r0 + STREAM) of a (rows, width) matrix into LDS at compute width, zero past
// `rows` and past `width`. Every load of the thread first, into registers, then the LDS writes:
// written as one loop, each element's load was waited for before its write, and the passes of a
// short head spent their time on one memory latency per staged element.
template <typename T, int MAXD>
__device__ __forceinline__ void stage(typename T::Compute (*tile)[row_stride<MAXD>()], const typename T::Storage* base, int64_t r0,
                                      int64_t rows, int width) {
  typedef typename T::Compute C;
  constexpr int STREAM = stream_rows<C, MAXD>(), N = STREAM * MAXD / THREADS;
  static_assert(N * THREADS == STREAM * MAXD, "a tile is a whole number of elements per thread");
  C vals[N];
#pragma unroll
  for (int n = 0; n < N; n++) {
    const int idx = threadIdx.x + n * THREADS;
    const int lr = idx / MAXD, d = idx - lr * MAXD;
    const int64_t r = r0 + lr;
    vals[n] = (r < rows && d < width) ? T::load(base, r * width + d) : C(0);
  }
#pragma unroll
  for (int n = 0; n < N; n++) {
    const int idx = threadIdx.x + n * THREADS;
    tile[idx / MAXD][idx % MAXD] = vals[n];
  }
}

// One row's vector of MAXD dims as this lane's MAXD / LANES share.
template <typename T, int MAXD>
__device__ __forceinline__ void load_row(typename T::Compute* dst, const typename T::Storage* base, int64_t row,
                                         bool valid, int width, int u) {
#pragma unroll
  for (int j = 0; j < MAXD / LANES; j++) {
    const int d = u + LANES * j;
    dst[j] = (valid && d < width) ? T::load(base, row * width + d) : typename T::Compute(0);
  }
}

template <typename T, int MAXD>
__device__ __forceinline__ void store_row(typename T::Storage* base, const typename T::Compute* src, int64_t row,
                                          int width, int u, typename T::Compute mul) {
#pragma unroll
  for (int j = 0; j < MAXD / LANES; j++) {
    const int d = u + LANES * j;
    if (d < width) T::store(base, row * width + d, src[j] * mul);
  }
}

template <typename T, int MAXD>
__device__ __forceinline__ typename T::Compute dot(const typename T::Compute* a, const typename T::Compute* lds_row, int u) {
  typename T::Compute s(0);
#pragma unroll
  for (int j = 0; j < MAXD / LANES; j++) s += a[j] * lds_row[u + LANES * j];
  return row_sum(s);
}

// the sum of x over the SPLIT key groups of a row (every group gets the total): lanes of one
// row's groups sit LANES apart
template <int SPLIT, typename C>
__device__ __forceinline__ C group_sum(C x) {
  if (SPLIT > 1) x += __shfl_xor(x, LANES);
  if (SPLIT > 2) x += __shfl_xor(x, 2 * LANES);
  if (SPLIT > 4) x += __shfl_xor(x, 4 * LANES);
  if (SPLIT > 8) x += __shfl_xor(x, 8 * LANES);
  return x;
}

template <int SPLIT, typename C>
__device__ __forceinline__ C group_max(C x) {
  if (SPLIT > 1) x = fmax(x, __shfl_xor(x, LANES));
  if (SPLIT > 2) x = fmax(x, __shfl_xor(x, 2 * LANES));
  if (SPLIT > 4) x = fmax(x, __shfl_xor(x, 4 * LANES));
  if (SPLIT > 8) x = fmax(x, __shfl_xor(x, 8 * LANES));
  return x;
}

template <typename T, int MAXD, int SPLIT>
__global__ __launch_bounds__(THREADS) void sdpa_fwd_rows(const typename T::Storage* __restrict__ q,
                                                         const typename T::Storage* __restrict__ k,
                                                         const typename T::Storage* __restrict__ v,
                                                         const typename T::Storage* __restrict__ mask,
                                                         typename T::Storage* __restrict__ out,
                                                         typename T::Compute* __restrict__ lse, int64_t t_q,
                                                         int64_t t_k, int hd, int hd_v, int causal,
                                                         typename T::Compute scale) {
  typedef typename T::Compute C;
  constexpr int P = MAXD / LANES, ROWS = rows_per_block<SPLIT>();
  constexpr int STREAM = stream_rows<C, MAXD>();
  __shared__ C Kt[STREAM][row_stride<MAXD>()];
  __shared__ C Vt[STREAM][row_stride<MAXD>()];
  __shared__ C Mt[STREAM];
  const int64_t chunks = (t_q + ROWS - 1) / ROWS;
  const int64_t b = blockIdx.x / chunks, chunk = blockIdx.x - b * chunks;
  const int u = threadIdx.x % LANES, grp = (threadIdx.x / LANES) % SPLIT;
  const int64_t i = chunk * ROWS + threadIdx.x / (LANES * SPLIT);
  const bool valid = i < t_q;
  C qv[P], acc[P];
  load_row<T, MAXD>(qv, q + b * t_q * hd, i, valid, hd, u);
#pragma unroll
  for (int j = 0; j < P; j++) acc[j] = C(0);
  C m = -__builtin_inf(), l = C(0);
  const int64_t keys_end = valid ? (causal ? i + 1 : t_k) : 0;
  const int64_t block_end = causal ? ((chunk + 1) * ROWS < t_k ? (chunk + 1) * ROWS : t_k) : t_k;
  for (int64_t r0 = 0; r0 < block_end; r0 += STREAM) {
    stage<T, MAXD>(Kt, k + b * t_k * hd, r0, t_k, hd);
    stage<T, MAXD>(Vt, v + b * t_k * hd_v, r0, t_k, hd_v);
    if (mask != nullptr && threadIdx.x < STREAM) {
      const int64_t r = r0 + threadIdx.x;
      Mt[threadIdx.x] = r < t_k ? T::load(mask, b * t_k + r) : C(0);
    }
    __syncthreads();
    const int64_t end = r0 + STREAM < keys_end ? r0 + STREAM : keys_end;
    for (int64_t j = r0 + grp; j < end; j += SPLIT) {
      const int lj = (int)(j - r0);
      if (mask != nullptr && Mt[lj] == C(0)) continue;
      const C s = dot<T, MAXD>(qv, Kt[lj], u) * scale;
      if (s > m) {
        const C alpha = exp_c<C>(m - s);
        l *= alpha;
#pragma unroll
        for (int e = 0; e < P; e++) acc[e] *= alpha;
        m = s;
      }
      const C p = exp_c<C>(s - m);
      l += p;
#pragma unroll
      for (int e = 0; e < P; e++) acc[e] += p * Vt[lj][u + LANES * e];
    }
    __syncthreads();
  }
  if (SPLIT > 1) {
    // the groups' totals rescaled to the row's max (a group that saw no visible key adds 0)
    const C mr = group_max<SPLIT>(m);
    const C f = m == -__builtin_inf() ? C(0) : exp_c<C>(m - mr);
    l = group_sum<SPLIT>(l * f);
#pragma unroll
    for (int e = 0; e < P; e++) acc[e] = group_sum<SPLIT>(acc[e] * f);
    m = mr;
  }
  if (valid && grp == 0) {
    store_row<T, MAXD>(out + b * t_q * hd_v, acc, i, hd_v, u, C(1) / l);
    if (u == 0) lse[b * t_q + i] = m + log_c<C>(l);
  }
}

template <typename T, int MAXD, int SPLIT>
__global__ __launch_bounds__(THREADS) void sdpa_bwd_q_rows(
    const typename T::Storage* __restrict__ q, const typename T::Storage* __restrict__ k,
    const typename T::Storage* __restrict__ v, const typename T::Storage* __restrict__ dout,
    const typename T::Compute* __restrict__ lse, const typename T::Compute* __restrict__ delta,
    const typename T::Storage* __restrict__ mask, typename T::Storage* __restrict__ dq, int64_t t_q, int64_t t_k, int hd,
    int hd_v, int causal, typename T::Compute scale) {
  typedef typename T::Compute C;
  constexpr int P = MAXD / LANES, ROWS = rows_per_block<SPLIT>();
  constexpr int STREAM = stream_rows<C, MAXD>();
  __shared__ C Kt[STREAM][row_stride<MAXD>()];
  __shared__ C Vt[STREAM][row_stride<MAXD>()];
  __shared__ C Mt[STREAM];
  const int64_t chunks = (t_q + ROWS - 1) / ROWS;
  const int64_t b = blockIdx.x / chunks, chunk = blockIdx.x - b * chunks;
  const int u = threadIdx.x % LANES, grp = (threadIdx.x / LANES) % SPLIT;
  const int64_t i = chunk * ROWS + threadIdx.x / (LANES * SPLIT);
  const bool valid = i < t_q;
  C qv[P], ov[P], g[P];
  load_row<T, MAXD>(qv, q + b * t_q * hd, i, valid, hd, u);
  load_row<T, MAXD>(ov, dout + b * t_q * hd_v, i, valid, hd_v, u);
#pragma unroll
  for (int e = 0; e < P; e++) g[e] = C(0);
  const C L = valid ? lse[b * t_q + i] : C(0);
  const C D = valid ? delta[b * t_q + i] : C(0);
  const int64_t keys_end = valid ? (causal ? i + 1 : t_k) : 0;
  const int64_t block_end = causal ? ((chunk + 1) * ROWS < t_k ? (chunk + 1) * ROWS : t_k) : t_k;
  for (int64_t r0 = 0; r0 < block_end; r0 += STREAM) {
    stage<T, MAXD>(Kt, k + b * t_k * hd, r0, t_k, hd);
    stage<T, MAXD>(Vt, v + b * t_k * hd_v, r0, t_k, hd_v);
    if (mask != nullptr && threadIdx.x < STREAM) {
      const int64_t r = r0 + threadIdx.x;
      Mt[threadIdx.x] = r < t_k ? T::load(mask, b * t_k + r) : C(0);
    }
    __syncthreads();
    const int64_t end = r0 + STREAM < keys_end ? r0 + STREAM : keys_end;
    for (int64_t j = r0 + grp; j < end; j += SPLIT) {
      const int lj = (int)(j - r0);
      if (mask != nullptr && Mt[lj] == C(0)) continue;
      const C s = dot<T, MAXD>(qv, Kt[lj], u);
      const C dp = dot<T, MAXD>(ov, Vt[lj], u);
      const C p = exp_c<C>(s * scale - L);
      const C ds = p * (dp - D) * scale;
#pragma unroll
      for (int e = 0; e < P; e++) g[e] += ds * Kt[lj][u + LANES * e];
    }
    __syncthreads();
  }
#pragma unroll
  for (int e = 0; e < P; e++) g[e] = group_sum<SPLIT>(g[e]);
  // a row whose every key is hidden has L = -inf: each of its probabilities is
  // exp(-inf - (-inf)) = NaN in the numpy reference (reference limn/sdpa.py:140-170), so its dQ is NaN
  if (L == -__builtin_inf()) {
#pragma unroll
    for (int e = 0; e < P; e++) g[e] = __builtin_nan("");
  }
  if (valid && grp == 0) store_row<T, MAXD>(dq + b * t_q * hd, g, i, hd, u, C(1));
}

template <typename T, int MAXD, int SPLIT>
__global__ __launch_bounds__(THREADS) void sdpa_bwd_kv_rows(
    const typename T::Storage* __restrict__ q, const typename T::Storage* __restrict__ k,
    const typename T::Storage* __restrict__ v, const typename T::Storage* __restrict__ dout,
    const typename T::Compute* __restrict__ lse, const typename T::Compute* __restrict__ delta,
    const typename T::Storage* __restrict__ mask, typename T::Storage* __restrict__ dk,
    typename T::Storage* __restrict__ dv, int64_t t_q, int64_t t_k, int hd, int hd_v, int causal,
    typename T::Compute scale) {
  typedef typename T::Compute C;
  constexpr int P = MAXD / LANES, ROWS = rows_per_block<SPLIT>();
  constexpr int STREAM = stream_rows<C, MAXD>();
  __shared__ C Qt[STREAM][row_stride<MAXD>()];
  __shared__ C Ot[STREAM][row_stride<MAXD>()];
  __shared__ C Lt[STREAM];
  __shared__ C Dt[STREAM];
  const int64_t chunks = (t_k + ROWS - 1) / ROWS;
  const int64_t b = blockIdx.x / chunks, chunk = blockIdx.x - b * chunks;
  const int u = threadIdx.x % LANES, grp = (threadIdx.x / LANES) % SPLIT;
  const int64_t j = chunk * ROWS + threadIdx.x / (LANES * SPLIT);
  const bool valid = j < t_k;
  const bool live = valid && (mask == nullptr || T::load(mask, b * t_k + j) != C(0));
  C kv[P], vv[P], gk[P], gv[P];
  load_row<T, MAXD>(kv, k + b * t_k * hd, j, valid, hd, u);
  load_row<T, MAXD>(vv, v + b * t_k * hd_v, j, valid, hd_v, u);
#pragma unroll
  for (int e = 0; e < P; e++) {
    gk[e] = C(0);
    gv[e] = C(0);
  }
  // a causal key j is seen by queries i >= j only, so the block starts at its own first key;
  // every thread meets the same barriers. A hidden key streams its queries too, with each
  // probability exp(-inf - L): zero, so its dK and dV stay exactly zero, except against a row
  // whose every key is hidden (L = -inf), where the numpy reference's probability is NaN
  // (reference limn/sdpa.py:173-203) and so are the key's gradients.
  const int64_t first = causal ? chunk * ROWS : 0;
  const int64_t rows_end = valid ? t_q : 0;
  for (int64_t r0 = first; r0 < t_q; r0 += STREAM) {
    stage<T, MAXD>(Qt, q + b * t_q * hd, r0, t_q, hd);
    stage<T, MAXD>(Ot, dout + b * t_q * hd_v, r0, t_q, hd_v);
    if (threadIdx.x < STREAM) {
      const int64_t r = r0 + threadIdx.x;
      Lt[threadIdx.x] = r < t_q ? lse[b * t_q + r] : C(0);
      Dt[threadIdx.x] = r < t_q ? delta[b * t_q + r] : C(0);
    }
    __syncthreads();
    const int64_t end = r0 + STREAM < rows_end ? r0 + STREAM : rows_end;
    // this group's queries of the tile: r0 + grp, r0 + grp + SPLIT, ..., from the key's own
    // position on under causality
    int64_t from = r0 + grp;
    if (causal && j > from) from += (j - from + SPLIT - 1) / SPLIT * SPLIT;
    for (int64_t i = from; i < end; i += SPLIT) {
      const int li = (int)(i - r0);
      const C s = dot<T, MAXD>(kv, Qt[li], u);
      const C dp = dot<T, MAXD>(vv, Ot[li], u);
      const C p = exp_c<C>((live ? s * scale : -__builtin_inf()) - Lt[li]);
      const C ds = p * (dp - Dt[li]) * scale;
#pragma unroll
      for (int e = 0; e < P; e++) {
        gv[e] += p * Ot[li][u + LANES * e];
        gk[e] += ds * Qt[li][u + LANES * e];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int e = 0; e < P; e++) {
    gk[e] = group_sum<SPLIT>(gk[e]);
    gv[e] = group_sum<SPLIT>(gv[e]);
  }
  if (valid && grp == 0) {
    store_row<T, MAXD>(dk + b * t_k * hd, gk, j, hd, u, C(1));
    store_row<T, MAXD>(dv + b * t_k * hd_v, gv, j, hd_v, u, C(1));
  }
}

template <typename T, int MAXD, int SPLIT>
int launch_rows(SdpaPass pass, const SdpaArgs& a) {
  typedef typename T::Storage S;
  typedef typename T::Compute C;
  constexpr int ROWS = rows_per_block<SPLIT>();
  const int64_t rows = pass == SDPA_BWD_KV ? a.t_k : a.t_q;
  const int64_t blocks = a.batch * ((rows + ROWS - 1) / ROWS);
  if (blocks > 0x7fffffff) return fail(LIMN_HIP_EUNSUPPORTED, "sdpa: %lld workgroups exceed one launch", (long long)blocks);
  const dim3 grid((unsigned)blocks), block(THREADS);
  const C scale = (C)a.scale;
  const int hd = (int)a.hd, hd_v = (int)a.hd_v, causal = a.causal ? 1 : 0;
  const S* mask = (const S*)a.mask;
  switch (pass) {
    case SDPA_FWD:
      hipLaunchKernelGGL((sdpa_fwd_rows<T, MAXD, SPLIT>), grid, block, 0, a.stream, (const S*)a.q, (const S*)a.k, (const S*)a.v,
                         mask, (S*)a.out0, (C*)a.out1, a.t_q, a.t_k, hd, hd_v, causal, scale);
      break;
    case SDPA_BWD_Q:
      hipLaunchKernelGGL((sdpa_bwd_q_rows<T, MAXD, SPLIT>), grid, block, 0, a.stream, (const S*)a.q, (const S*)a.k,
                         (const S*)a.v, (const S*)a.dout, (const C*)a.lse, (const C*)a.delta, mask, (S*)a.out0, a.t_q,
                         a.t_k, hd, hd_v, causal, scale);
      break;
    case SDPA_BWD_KV:
      hipLaunchKernelGGL((sdpa_bwd_kv_rows<T, MAXD, SPLIT>), grid, block, 0, a.stream, (const S*)a.q, (const S*)a.k,
                         (const S*)a.v, (const S*)a.dout, (const C*)a.lse, (const C*)a.delta, mask, (S*)a.out0,
                         (S*)a.out1, a.t_q, a.t_k, hd, hd_v, causal, scale);
      break;
  }
  return check_hip(hipGetLastError(), "launching an sdpa kernel");
}

// split each row's streamed rows among 4, 8 or 16 groups of lanes when whole rows per lane
// group would leave most CUs without a workgroup
template <typename T, int MAXD>
int launch_split(SdpaPass pass, const SdpaArgs& a) {
  const int64_t rows = pass == SDPA_BWD_KV ? a.t_k : a.t_q;
  const int64_t whole = a.batch * ((rows + rows_per_block<1>() - 1) / rows_per_block<1>());
  if (whole < 64) return launch_rows<T, MAXD, 16>(pass, a);
  if (whole < 256) return launch_rows<T, MAXD, 8>(pass, a);
  if (whole < 1024) return launch_rows<T, MAXD, 4>(pass, a);
  return launch_rows<T, MAXD, 1>(pass, a);
}

template <typename T>
int launch_width(SdpaPass pass, const SdpaArgs& a) {
  const int64_t width = a.hd > a.hd_v ? a.hd : a.hd_v;
  if (width <= 16) return launch_split<T, 16>(pass, a);
  if (width <= 64) return launch_split<T, 64>(pass, a);
  if (width <= 128) return launch_split<T, 128>(pass, a);
  return launch_split<T, 256>(pass, a);
}

}  // namespace

bool rows_supports(int dtype, int64_t hd, int64_t hd_v) {
  const bool known = dtype == LIMN_HIP_FLOAT64 || dtype == LIMN_HIP_FLOAT32 || dtype == LIMN_HIP_FLOAT16 ||
                     dtype == LIMN_HIP_BFLOAT16;
  return known && hd >= 1 && hd_v >= 1 && hd <= 256 && hd_v <= 256;
}

int launch_sdpa_rows(SdpaPass pass, const SdpaArgs& a) {
  switch (a.dtype) {
    case LIMN_HIP_FLOAT64:
      return launch_width<F64>(pass, a);
    case LIMN_HIP_FLOAT32:
      return launch_width<F32>(pass, a);
    case LIMN_HIP_FLOAT16:
      return launch_width<F16>(pass, a);
    case LIMN_HIP_BFLOAT16:
      return launch_width<BF16>(pass, a);
  }
  return fail(LIMN_HIP_EUNSUPPORTED, "sdpa: unknown dtype code %d", a.dtype);
}

}  // namespace limn
