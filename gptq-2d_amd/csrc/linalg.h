// Internal dense linear-algebra launchers shared by the LDL preprocessing (ldl.hip) and
// built on the strided GEMM of gemm.hip.  Not part of the C ABI.
#pragma once

#include "common.h"

// Structure of an operand: which of its entries may be non-zero.  The kernels never read the
// structurally zero part, so it may hold anything (the other triangle of a factor, NaN, ...).
enum TriMode : int32_t {
  TRI_NONE = 0,
  TRI_LOWER = 1,  // entry (r, c) is zero for c > r
  TRI_UPPER = 2,  // entry (r, c) is zero for c < r
};

// D(i, j) = beta * D(i, j) + alpha * sum_k A(i, k) B(k, j) over i < M, j < N, k < K, for `batch`
// independent problems.  X(r, c) = X[batch_index * x_bs + r * x_rs + c * x_cs] for X in A, B, D
// (any strides: transposed and reversed views are free).  beta == 0 never reads D.  d_tri
// restricts the written entries (TRI_LOWER: i >= j only).
template <typename T>
struct GemmProblem {
  int64_t M, N, K, batch;
  const T* A;
  int64_t a_rs, a_cs, a_bs;
  const T* B;
  int64_t b_rs, b_cs, b_bs;
  T* D;
  int64_t d_rs, d_cs, d_bs;
  T alpha, beta;
  int32_t a_tri, b_tri, d_tri;
};

template <typename T>
int gptq2d_gemm(const GemmProblem<T>& p, hipStream_t stream);

// Row-major fp32 D = alpha A B (no beta) for `batch` strided problems with one lower triangular
// operand whose other triangle holds zeros: tri = 1: B (B(k, j) = 0 for k < j), tri = 2: A
// (A(i, k) = 0 for k > i), 0: dense.  A: M x K (row stride lda, batch stride sa), B: K x N, D: M x N.
// On MFMA, skipping the k-tiles that meet only the zero triangle (trmm_mfma.hip).  Needs K, N, lda,
// ldb, sa, sb multiples of 4, A and B on 16-byte boundaries and each operand under 2^29 elements;
// returns GPTQ2D_EUNSUPPORTED otherwise (nothing launched).
struct TriGemm {
  int64_t M, N, K, batch;
  const float* A;
  int64_t lda, sa;
  const float* B;
  int64_t ldb, sb;
  float* D;
  int64_t ldd, sd;
  float alpha;
  int32_t tri;
  // a second batch dimension (0 or 1: none): problem (y, z) at A + y sa + z sa2, and so on
  int64_t batch2, sa2, sb2, sd2;
};

int gptq2d_tri_gemm_f32(const TriGemm& g, hipStream_t stream);
