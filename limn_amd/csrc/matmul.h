// Internal launch interface of the dense-contraction kernel (matmul.hip).
#pragma once

#include "common.h"

namespace limn {

// C[b, m, n] = sum_k A[b, m, k] * B[b, k, n]; all strides in elements.
struct MatmulShape {
  int64_t batch, M, N, K;
  int64_t a_batch, a_m, a_k;
  int64_t b_batch, b_k, b_n;
  int64_t c_batch, c_m, c_n;
};

enum { MATMUL_EPILOGUE_NONE = 0, MATMUL_EPILOGUE_RELU = 1 };

// Terms added to the contraction after it is rounded to the output type, with one more rounding
// at the end: out = T(res[b, m, n] + (T(epilogue(sum)) + bias[n])), computed in float, either term
// left out when its pointer is null. This is an elementwise reader of the contraction that adds a
// bias vector (and a residual), evaluated at the store instead of in a launch of its own.
struct MatmulAddends {
  const void* bias;  // bias[n * bias_n], of the output type, or float32 rounded to it first
  int bias_f32;
  int64_t bias_n;
  const u16* res;   // res[b * r_batch + m * r_m + n * r_n]
  int64_t r_batch, r_m, r_n;
  int vec;          // bit 0: bias_n == 1 and 16-byte aligned; bit 1: res rows the same (r_n == 1)
};

// How a contraction is cut: output tiles of `tile` x `tile`, k in `split` slices of `chunk`.
struct MatmulPlan {
  int tile;
  int64_t split, chunk;
};
MatmulPlan plan_matmul(const MatmulShape& s);
int64_t matmul_workspace_bytes(const MatmulShape& s);

// 1 when every operand is contiguous along one of its two dims with 16-byte aligned rows.
int matmul_layout_ok(const MatmulShape& s);
int launch_matmul(const void* a, const void* b, void* c, int dtype, const MatmulShape& s, int epilogue,
                  const MatmulAddends& add, void* workspace, int64_t workspace_bytes, hipStream_t stream);

}  // namespace limn
