// Block flush of the GPTQ-2D sweep: the errors of a finished band of stages reach all target
// entries of later stages through two masked band GEMMs, fused in one kernel.
//
// Stages are coarse antidiagonals i/P + j/Q (P = Q = 1 for plain entries, the super-entry shape
// for super-entries, the tile shape for the fused tile sweep).  For the band of stages
// [s0, s1) and every target (i, j) with s1 <= i/P + j/Q < s_end:
//
//   D[i,j] = sum_k L[i,k] E[k,j]   over s0 <= k/P + j/Q < s1, k/P < i/P   (down, through L)
//   R[i,j] = sum_k C[i,k] U[k,j]   over s0 <= i/P + k/Q < s1, k/Q < j/Q   (right, through U)
//   C[i,j] += D[i,j];  Y[i,j] = (Y[i,j] + D[i,j]) + R[i,j]
//
// The right product reads C only on the band, which the down product never writes (it writes
// targets only), so both run in one pass per output tile with a single read-modify-write of Y and C.
// L is read only strictly below its P x P diagonal blocks and U strictly above its Q x Q ones;
// masked loads never touch other entries (they may hold NaN).
//
// Reference counterparts (IST-DASLab/GPTQ-2D, gptq_2d.py): _repack_errors_kernel :633-737,
// _flush_down_kernel :766-902 and _flush_right_kernel :936-1057, applied in that order by
// _flush_block :1090-1119.  The band of E is read in matrix layout with a mask, so no repack.
#include "common.h"
#include "profile.h"

namespace {

constexpr int FB_M = 64, FB_N = 64, FB_K = 16;

struct FlushGeom {
  int64_t m, n, P, Q, s0, s1, s_end;
};

// Column-tile range of target tile row ti (rows i0..i1-1), by output tile width FB_N.
__host__ __device__ inline void target_cols(const FlushGeom& g, int64_t i0, int64_t i1, int64_t& jt_lo,
                                            int64_t& jt_hi) {
  const int64_t cb_lo = g.s1 - (i1 - 1) / g.P;  // smallest coarse target column in these rows
  const int64_t cb_hi = g.s_end - 1 - i0 / g.P;  // largest
  int64_t j_lo = cb_lo * g.Q;
  if (j_lo < 0) j_lo = 0;
  int64_t j_hi = (cb_hi + 1) * g.Q;
  if (j_hi > g.n) j_hi = g.n;
  if (cb_hi < 0 || j_hi <= j_lo) {
    jt_lo = jt_hi = 0;
    return;
  }
  jt_lo = j_lo / FB_N;
  jt_hi = (j_hi + FB_N - 1) / FB_N;
}

template <typename T>
__global__ __launch_bounds__(256) void flush_valu_kernel(T* __restrict__ y, T* __restrict__ c,
                                                         const T* __restrict__ e, const T* __restrict__ l,
                                                         const T* __restrict__ u, FlushGeom g, BatchMap lmap,
                                                         BatchMap umap, int64_t nx, int64_t ny) {
  __shared__ T As[FB_K][FB_M + 1];
  __shared__ T Bs[FB_K][FB_N + 1];
  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t m = g.m, n = g.n, P = g.P, Q = g.Q;
  const int64_t i0 = id.y * FB_M;
  const int64_t i1 = i0 + FB_M < m ? i0 + FB_M : m;
  int64_t jt_lo, jt_hi;
  target_cols(g, i0, i1, jt_lo, jt_hi);
  const int64_t jt = jt_lo + id.x;
  if (jt >= jt_hi) return;
  const int64_t j0 = jt * FB_N;
  const int64_t j1 = j0 + FB_N < n ? j0 + FB_N : n;
  // whole tile outside the targets?
  if ((i1 - 1) / P + (j1 - 1) / Q < g.s1 || i0 / P + j0 / Q >= g.s_end) return;

  const int tid = threadIdx.x;
  const int tx = tid & 15, ty = tid >> 4;
  const int64_t mat = b * m * n;
  const T* lb = l + lmap.offset(b);
  const T* ub = u + umap.offset(b);

  T accd[4][4], accr[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2) accd[a][q2] = accr[a][q2] = T(0);

  // ---------------- down: D = L E over the band (only columns j < s1*Q have band rows)
  if (j0 / Q < g.s1) {
    int64_t k_lo = (g.s0 - (j1 - 1) / Q) * P;
    if (k_lo < 0) k_lo = 0;
    int64_t k_hi = (g.s1 - j0 / Q) * P;
    const int64_t k_cap = ((i1 - 1) / P) * P;  // L strictly below diagonal blocks
    if (k_hi > k_cap) k_hi = k_cap;
    if (k_hi > m) k_hi = m;
    for (int64_t kb = k_lo; kb < k_hi; kb += FB_K) {
      // A = L[i, k]: thread t loads k = kb + t%16, i = i0 + t/16 + 16*ld
#pragma unroll
      for (int ld = 0; ld < 4; ++ld) {
        const int kl = tid & 15, il = (tid >> 4) + 16 * ld;
        const int64_t i = i0 + il, k = kb + kl;
        T v = T(0);
        if (i < i1 && k < k_hi && k / P < i / P) v = lb[i * m + k];
        As[kl][il] = v;
      }
      // B = E[k, j] on the band: thread t loads j = j0 + t%64, k = kb + t/64 + 4*ld
#pragma unroll
      for (int ld = 0; ld < 4; ++ld) {
        const int jl = tid & 63, kl = (tid >> 6) + 4 * ld;
        const int64_t j = j0 + jl, k = kb + kl;
        T v = T(0);
        if (j < j1 && k < k_hi) {
          const int64_t st = k / P + j / Q;
          if (st >= g.s0 && st < g.s1) v = e[mat + k * n + j];
        }
        Bs[kl][jl] = v;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < FB_K; ++kk) {
        T av[4], bv[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) av[a] = As[kk][ty + 16 * a];
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) bv[q2] = Bs[kk][tx + 16 * q2];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int q2 = 0; q2 < 4; ++q2) accd[a][q2] += av[a] * bv[q2];
      }
      __syncthreads();
    }
  }

  // ---------------- right: R = C U over the band (only rows i < s1*P have band columns)
  if (i0 / P < g.s1) {
    int64_t k_lo = (g.s0 - (i1 - 1) / P) * Q;
    if (k_lo < 0) k_lo = 0;
    int64_t k_hi = (g.s1 - i0 / P) * Q;
    const int64_t k_cap = ((j1 - 1) / Q) * Q;  // U strictly above diagonal blocks
    if (k_hi > k_cap) k_hi = k_cap;
    if (k_hi > n) k_hi = n;
    for (int64_t kb = k_lo; kb < k_hi; kb += FB_K) {
      // A = C[i, k] on the band
#pragma unroll
      for (int ld = 0; ld < 4; ++ld) {
        const int kl = tid & 15, il = (tid >> 4) + 16 * ld;
        const int64_t i = i0 + il, k = kb + kl;
        T v = T(0);
        if (i < i1 && k < k_hi) {
          const int64_t st = i / P + k / Q;
          if (st >= g.s0 && st < g.s1) v = c[mat + i * n + k];
        }
        As[kl][il] = v;
      }
      // B = U[k, j] strictly above diagonal blocks
#pragma unroll
      for (int ld = 0; ld < 4; ++ld) {
        const int jl = tid & 63, kl = (tid >> 6) + 4 * ld;
        const int64_t j = j0 + jl, k = kb + kl;
        T v = T(0);
        if (j < j1 && k < k_hi && k / Q < j / Q) v = ub[k * n + j];
        Bs[kl][jl] = v;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < FB_K; ++kk) {
        T av[4], bv[4];
#pragma unroll
        for (int a = 0; a < 4; ++a) av[a] = As[kk][ty + 16 * a];
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) bv[q2] = Bs[kk][tx + 16 * q2];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
          for (int q2 = 0; q2 < 4; ++q2) accr[a][q2] += av[a] * bv[q2];
      }
      __syncthreads();
    }
  }

  // ---------------- epilogue: only the targets receive the feedback
#pragma unroll
  for (int a = 0; a < 4; ++a) {
    const int64_t i = i0 + ty + 16 * a;
    if (i >= i1) continue;
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2) {
      const int64_t j = j0 + tx + 16 * q2;
      if (j >= j1) continue;
      const int64_t st = i / P + j / Q;
      if (st < g.s1 || st >= g.s_end) continue;
      const int64_t off = mat + i * n + j;
      c[off] = c[off] + accd[a][q2];
      y[off] = (y[off] + accd[a][q2]) + accr[a][q2];
    }
  }
}

}  // namespace

// Grid over the target band: y = output tile row, x = column tile within that row's target range.
static int64_t flush_grid_x(const FlushGeom& g, int64_t& nrow_tiles) {
  const int64_t rows = g.s_end * g.P < g.m ? g.s_end * g.P : g.m;
  nrow_tiles = cdiv(rows, FB_M);
  int64_t nx = 0;
  for (int64_t ti = 0; ti < nrow_tiles; ++ti) {
    const int64_t i0 = ti * FB_M, i1 = i0 + FB_M < g.m ? i0 + FB_M : g.m;
    int64_t lo, hi;
    target_cols(g, i0, i1, lo, hi);
    if (hi - lo > nx) nx = hi - lo;
  }
  return nx;
}

// Useful flops of one flush: 2 per (target, source) pair that the two band products sum, i.e.
// for a coarse target cell (a, b) of h(a) x w(b) entries, 2 h(a) w(b) (sum of h(a') over the down
// sources a' + sum of w(b') over the right sources b').  Host-side, for the launch profiler.
double gptq2d_flush_flops(int64_t m, int64_t n, int64_t P, int64_t Q, int64_t s0, int64_t s1, int64_t s_end) {
  const int64_t mc = cdiv(m, P), nc = cdiv(n, Q);
  auto h = [&](int64_t a) { return (double)((a + 1) * P < m ? P : m - a * P); };
  auto w = [&](int64_t b) { return (double)((b + 1) * Q < n ? Q : n - b * Q); };
  double total = 0.;
  for (int64_t a = 0; a < mc; ++a) {
    for (int64_t b = s1 - a > 0 ? s1 - a : 0; b < nc && a + b < s_end; ++b) {
      double rows = 0., cols = 0.;
      for (int64_t a2 = s0 - b > 0 ? s0 - b : 0; a2 < s1 - b && a2 < a; ++a2) rows += h(a2);
      for (int64_t b2 = s0 - a > 0 ? s0 - a : 0; b2 < s1 - a && b2 < b; ++b2) cols += w(b2);
      total += 2. * h(a) * w(b) * (rows + cols);
    }
  }
  return total;
}

int gptq2d_flush_tiles_mfma(float* y, float* c, const float* e, const float* l, const float* u, int64_t m, int64_t n,
                            int64_t S0, int64_t S1, int64_t S_end, const BatchMap& lmap, const BatchMap& umap,
                            int64_t B, hipStream_t stream);

template <typename T>
int gptq2d_flush(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t P, int64_t Q,
                 int64_t s0, int64_t s1, int64_t s_end, const BatchMap& lmap, const BatchMap& umap, int64_t B,
                 hipStream_t stream) {
  if (m <= 0 || n <= 0 || P <= 0 || Q <= 0 || s0 < 0 || s1 <= s0 || s_end < s1) return GPTQ2D_EINVAL;
  if (B == 0 || s_end == s1) return 0;
  if constexpr (sizeof(T) == 4) {
    // 32 x 32 coarse cells (the fused engine's tiles, or 32 x 32 super-entries): fp32 MFMA (its buffer
    // resources are based at each panel, so 32-bit offsets hold for rows and k-tiles of up to 2^20
    // elements, i.e. any m, n < 2^20)
    if (P == 32 && Q == 32 && m < ((int64_t)1 << 20) && n < ((int64_t)1 << 20)) {
      const bool prof = gptq2d_prof_on(PROF_FLUSH);
      if (prof) gptq2d_prof_begin(PROF_FLUSH, stream);
      const int rc = gptq2d_flush_tiles_mfma(y, c, e, l, u, m, n, s0, s1, s_end, lmap, umap, B, stream);
      if (prof) gptq2d_prof_end(PROF_FLUSH, (double)B * gptq2d_flush_flops(m, n, P, Q, s0, s1, s_end), stream);
      return rc;
    }
  }
  FlushGeom g{m, n, P, Q, s0, s1, s_end};
  int64_t nrow_tiles;
  const int64_t nx = flush_grid_x(g, nrow_tiles);
  if (nx == 0 || nrow_tiles == 0) return 0;
  Grid3 gr = make_grid(nx, nrow_tiles, B);
  const bool prof = gptq2d_prof_on(PROF_FLUSH);
  if (prof) gptq2d_prof_begin(PROF_FLUSH, stream);
  hipLaunchKernelGGL(flush_valu_kernel<T>, gr.grid, dim3(256), 0, stream, y, c, e, l, u, g, lmap, umap, gr.nx, gr.ny);
  if (prof) gptq2d_prof_end(PROF_FLUSH, (double)B * gptq2d_flush_flops(m, n, P, Q, s0, s1, s_end), stream);
  return (int)hipGetLastError();
}

template int gptq2d_flush<float>(float*, float*, const float*, const float*, const float*, int64_t, int64_t, int64_t,
                                 int64_t, int64_t, int64_t, int64_t, const BatchMap&, const BatchMap&, int64_t,
                                 hipStream_t);
template int gptq2d_flush<double>(double*, double*, const double*, const double*, const double*, int64_t, int64_t,
                                  int64_t, int64_t, int64_t, int64_t, int64_t, const BatchMap&, const BatchMap&,
                                  int64_t, hipStream_t);

extern "C" {

#define GPTQ2D_FLUSH_ABI(SUF, T)                                                                                    \
  int gptq2d_flush_##SUF(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t p,          \
                         int64_t q, int64_t s0, int64_t s1, int64_t s_end, int32_t bnd, const int64_t* bshape,      \
                         const int64_t* lstride, const int64_t* ustride, hipStream_t stream) {                      \
    BatchMap lmap, umap;                                                                                            \
    if (!make_batch_map(lmap, bnd, bshape, lstride) || !make_batch_map(umap, bnd, bshape, ustride))                 \
      return GPTQ2D_EINVAL;                                                                                         \
    return gptq2d_flush<T>(y, c, e, l, u, m, n, p, q, s0, s1, s_end, lmap, umap, batch_count(bnd, bshape), stream); \
  }

GPTQ2D_FLUSH_ABI(f32, float)
GPTQ2D_FLUSH_ABI(f64, double)

}  // extern "C"
