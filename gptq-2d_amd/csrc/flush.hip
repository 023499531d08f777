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
// Both products run on MFMA: 32 x 32 cells (the fused engine's tiles) on the tuned kernel of flush_mfma.hip
// (fp32; fp64 with even m and n), every other cell shape on flush_mfma_kernel here (16 x 16 x 4 MFMA, entries
// masked one by one at staging, so any P and Q).
// L is read only strictly below its P x P diagonal blocks and U strictly above its Q x Q ones;
// masked loads never touch other entries (they may hold NaN).
//
// Reference counterparts (IST-DASLab/GPTQ-2D, gptq_2d.py): _repack_errors_kernel :633-737,
// _flush_down_kernel :766-902 and _flush_right_kernel :936-1057, applied in that order by
// _flush_block :1090-1119.  The band of E is read in matrix layout with a mask, so no repack.
#include "common.h"
#include "profile.h"

namespace {

constexpr int FB_M = 64, FB_N = 64, FB_K = 32;

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

// MFMA operand and accumulator types of the 16 x 16 x 4 products.  In both v_mfma_f32_16x16x4f32 and
// v_mfma_f64_16x16x4f64 lane l supplies A(l % 16, l / 16) and B(l / 16, l % 16); accumulator element r of
// lane l holds D(row(l / 16, r), l % 16) with row = 4 (l / 16) + r for fp32 and l / 16 + 4 r for fp64
// (measured with a one-wave probe of each instruction).
template <typename T>
struct Mfma16;
template <>
struct Mfma16<float> {
  typedef float acc_t __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ acc_t mma(float a, float b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int kq, int r) { return 4 * kq + r; }
};
template <>
struct Mfma16<double> {
  typedef double acc_t __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ acc_t mma(double a, double b, acc_t c) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ int row(int kq, int r) { return kq + 4 * r; }
};

// LDS pitch of the staged panels (elements per k-row of FB_M or FB_N entries): a half-wave's MFMA operand
// read spans two k-rows of 16 entries, which the pad of 16 puts on disjoint banks.
constexpr int FB_P = FB_M + 16;

// The flush of one FB_M x FB_N output tile on MFMA: the two masked band products of FB_K-deep k-blocks
// staged in LDS, wave w computing the 32 x 32 quadrant (w / 2, w % 2) as 2 x 2 blocks of 16 x 16 x 4
// products, D and R in their own accumulators; then C += D and Y = (Y + D) + R on the targets.  Every
// staged operand entry is masked to what its product may read -- L strictly below its P x P diagonal
// blocks, U strictly above its Q x Q ones, E and C on the band, nothing outside the matrix -- through k
// limits that a staging thread computes once for each of its rows or columns (a row i of L is read for k
// below P floor(i / P); a column j of E for k in [P (s0 - floor(j / Q)), P (s1 - floor(j / Q))); and the
// same with the roles of P and Q exchanged for C and U), so that no division runs in the k loop.
template <typename T>
__global__ __launch_bounds__(256) void flush_mfma_kernel(T* __restrict__ y, T* __restrict__ c,
                                                         const T* __restrict__ e, const T* __restrict__ l,
                                                         const T* __restrict__ u, FlushGeom g, BatchMap lmap,
                                                         BatchMap umap, int64_t nx, int64_t ny) {
  using M = Mfma16<T>;
  using acc_t = typename M::acc_t;
  constexpr int AL = FB_M * FB_K / 256;  // staged entries per thread and operand
  __shared__ T As[FB_K][FB_P];
  __shared__ T Bs[FB_K][FB_P];
  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t m = g.m, n = g.n;
  const int64_t i0 = id.y * FB_M;
  const int64_t i1 = i0 + FB_M < m ? i0 + FB_M : m;
  int64_t jt_lo, jt_hi;
  target_cols(g, i0, i1, jt_lo, jt_hi);
  const int64_t jt = jt_lo + id.x;
  if (jt >= jt_hi) return;
  const int64_t j0 = jt * FB_N;
  const int64_t j1 = j0 + FB_N < n ? j0 + FB_N : n;
  // whole tile outside the targets?
  if ((i1 - 1) / g.P + (j1 - 1) / g.Q < g.s1 || i0 / g.P + j0 / g.Q >= g.s_end) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kq = lane >> 4;                 // operand row / column in a block, k in a 4-step
  const int wi = 32 * (wave >> 1), wj = 32 * (wave & 1);    // the wave's quadrant
  // staging roles: A entry x of this thread is (row ar + (256 / FB_K) x, k-offset ak); B entry x is
  // (k-offset bk + (256 / FB_N) x, column bj)
  constexpr int ASTEP = 256 / FB_K, BSTEP = 256 / FB_N;
  const int ak = tid % FB_K, ar = tid / FB_K;
  const int bj = tid % FB_N, bk = tid / FB_N;
  const int64_t P = g.P, Q = g.Q, s0 = g.s0, s1 = g.s1;
  // a k limit clamped into [0, k_hi] (so that it fits 32 bits like every k)
  auto clampk = [](int64_t v, int64_t k_hi) { return (int)(v < 0 ? 0 : (v < k_hi ? v : k_hi)); };
  const int64_t mat = b * m * n;
  const T* lb = l + lmap.offset(b);
  const T* ub = u + umap.offset(b);

  acc_t accd[2][2], accr[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 4; ++r) accd[a][d][r] = accr[a][d][r] = T(0);

  // the staged k-block's products into acc: FB_K / 4 steps of 4 k, 2 x 2 blocks
  auto mma_block = [&](acc_t (&acc)[2][2]) {
#pragma unroll
    for (int k4 = 0; k4 < FB_K; k4 += 4) {
      T av[2], bv[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) av[a] = As[k4 + kq][wi + 16 * a + li];
#pragma unroll
      for (int d = 0; d < 2; ++d) bv[d] = Bs[k4 + kq][wj + 16 * d + li];
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int d = 0; d < 2; ++d) acc[a][d] = M::mma(av[a], bv[d], acc[a][d]);
    }
  };

  // one band product: A rows from arow[x] (k limits [alo[x], ahi[x])), B columns from bcol (k limits
  // [blo, bhi)), k-blocks from k_lo up to k_hi; operand entries outside their limits are staged as zero
  // (the next k-block's entries are loaded into registers while the current one's MFMAs run)
  auto product = [&](acc_t (&acc)[2][2], const T* const (&arow)[AL], const int (&alo)[AL], const int (&ahi)[AL],
                     const T* bcol, int64_t bld, int blo, int bhi, int64_t k_lo, int64_t k_hi) {
    T ra[AL], rb[AL];
    auto load = [&](int64_t kb) {
      const int ka = (int)kb + ak;
#pragma unroll
      for (int x = 0; x < AL; ++x) ra[x] = (ka >= alo[x] && ka < ahi[x]) ? arow[x][ka] : T(0);
#pragma unroll
      for (int x = 0; x < AL; ++x) {
        const int kr = (int)kb + bk + BSTEP * x;
        rb[x] = (kr >= blo && kr < bhi) ? bcol[(int64_t)kr * bld] : T(0);
      }
    };
    if (k_lo < k_hi) load(k_lo);
    for (int64_t kb = k_lo; kb < k_hi; kb += FB_K) {
#pragma unroll
      for (int x = 0; x < AL; ++x) {
        As[ak][ar + ASTEP * x] = ra[x];
        Bs[bk + BSTEP * x][bj] = rb[x];
      }
      __syncthreads();
      if (kb + FB_K < k_hi) load(kb + FB_K);
      mma_block(acc);
      __syncthreads();
    }
  };

  // ---------------- down: D = L E over the band (only columns j < s1*Q have band rows)
  if (j0 / g.Q < g.s1) {
    int64_t k_lo = (g.s0 - (j1 - 1) / g.Q) * g.P;
    if (k_lo < 0) k_lo = 0;
    int64_t k_hi = (g.s1 - j0 / g.Q) * g.P;
    const int64_t k_cap = ((i1 - 1) / g.P) * g.P;  // L strictly below diagonal blocks
    if (k_hi > k_cap) k_hi = k_cap;
    if (k_hi > m) k_hi = m;
    const T* arow[AL];
    int alo[AL], ahi[AL];
#pragma unroll
    for (int x = 0; x < AL; ++x) {
      const int64_t i = i0 + ar + ASTEP * x;
      const bool in = i < i1;
      arow[x] = lb + (in ? i : 0) * m;
      alo[x] = 0;
      ahi[x] = in ? clampk(i / P * P, k_hi) : 0;  // k / P < i / P
    }
    const int64_t j = j0 + bj;
    int blo = 0, bhi = 0;
    if (j < j1) {  // s0 <= k / P + j / Q < s1
      blo = clampk((s0 - j / Q) * P, k_hi);
      bhi = clampk((s1 - j / Q) * P, k_hi);
    }
    product(accd, arow, alo, ahi, e + mat + (j < j1 ? j : 0), n, blo, bhi, k_lo, k_hi);
  }

  // ---------------- right: R = C U over the band (only rows i < s1*P have band columns)
  if (i0 / g.P < g.s1) {
    int64_t k_lo = (g.s0 - (i1 - 1) / g.P) * g.Q;
    if (k_lo < 0) k_lo = 0;
    int64_t k_hi = (g.s1 - i0 / g.P) * g.Q;
    const int64_t k_cap = ((j1 - 1) / g.Q) * g.Q;  // U strictly above diagonal blocks
    if (k_hi > k_cap) k_hi = k_cap;
    if (k_hi > n) k_hi = n;
    const T* arow[AL];
    int alo[AL], ahi[AL];
#pragma unroll
    for (int x = 0; x < AL; ++x) {
      const int64_t i = i0 + ar + ASTEP * x;
      const bool in = i < i1;
      arow[x] = c + mat + (in ? i : 0) * n;
      alo[x] = clampk((s0 - i / P) * Q, k_hi);  // s0 <= i / P + k / Q < s1
      ahi[x] = in ? clampk((s1 - i / P) * Q, k_hi) : 0;
    }
    const int64_t j = j0 + bj;
    const int bhi = j < j1 ? clampk(j / Q * Q, k_hi) : 0;  // k / Q < j / Q
    product(accr, arow, alo, ahi, ub + (j < j1 ? j : 0), n, 0, bhi, k_lo, k_hi);
  }

  // ---------------- epilogue: only the targets receive the feedback.  Every load of C and Y first, then the
  // new values, then the stores: entry by entry, each load would wait behind the previous entry's stores
  // (the compiler cannot prove the entries distinct), one memory round trip per entry and matrix.
  T cv[2][2][4], yv[2][2][4];
  uint32_t ok = 0;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const int64_t j = j0 + wj + 16 * d + li;
    const int64_t jc = j / g.Q;
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t i = i0 + wi + 16 * a + M::row(kq, r);
        const int64_t st = i / g.P + jc;
        cv[a][d][r] = yv[a][d][r] = T(0);
        if (j < j1 && i < i1 && st >= g.s1 && st < g.s_end) {
          ok |= 1u << (8 * d + 4 * a + r);
          const int64_t off = mat + i * n + j;
          cv[a][d][r] = c[off];
          yv[a][d][r] = y[off];
        }
      }
  }
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        cv[a][d][r] = cv[a][d][r] + accd[a][d][r];
        yv[a][d][r] = (yv[a][d][r] + accd[a][d][r]) + accr[a][d][r];
        asm volatile("" : "+v"(cv[a][d][r]), "+v"(yv[a][d][r]));  // here, not inside the stores' branches
      }
#pragma unroll
  for (int d = 0; d < 2; ++d)
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if ((ok >> (8 * d + 4 * a + r)) & 1) {
          const int64_t off = mat + (i0 + wi + 16 * a + M::row(kq, r)) * n + (j0 + wj + 16 * d + li);
          c[off] = cv[a][d][r];
          y[off] = yv[a][d][r];
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

template <typename T>
bool gptq2d_flush_tiles_mfma_fits(const T* y, const T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n,
                                  const BatchMap& lmap, const BatchMap& umap);
template <typename T>
int gptq2d_flush_tiles_mfma(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t S0,
                            int64_t S1, int64_t S_end, const BatchMap& lmap, const BatchMap& umap, int64_t B,
                            hipStream_t stream);

template <typename T>
int gptq2d_flush(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t P, int64_t Q,
                 int64_t s0, int64_t s1, int64_t s_end, const BatchMap& lmap, const BatchMap& umap, int64_t B,
                 hipStream_t stream) {
  if (m <= 0 || n <= 0 || P <= 0 || Q <= 0 || s0 < 0 || s1 <= s0 || s_end < s1) return GPTQ2D_EINVAL;
  if (B == 0 || s_end == s1) return 0;
  // 32 x 32 coarse cells (the fused engine's tiles, or 32 x 32 super-entries): the tuned kernel of
  // flush_mfma.hip where its size and alignment limits allow (fp32: m, n < 2^20; fp64 also m, n even and
  // 16-byte aligned matrices); everything else on the cell-masked MFMA kernel below
  if (P == 32 && Q == 32 && gptq2d_flush_tiles_mfma_fits<T>(y, c, e, l, u, m, n, lmap, umap)) {
    const bool prof = gptq2d_prof_on(PROF_FLUSH);
    if (prof) gptq2d_prof_begin(PROF_FLUSH, stream);
    const int rc = gptq2d_flush_tiles_mfma<T>(y, c, e, l, u, m, n, s0, s1, s_end, lmap, umap, B, stream);
    if (prof) gptq2d_prof_end(PROF_FLUSH, (double)B * gptq2d_flush_flops(m, n, P, Q, s0, s1, s_end), stream);
    return rc;
  }
  FlushGeom g{m, n, P, Q, s0, s1, s_end};
  int64_t nrow_tiles;
  const int64_t nx = flush_grid_x(g, nrow_tiles);
  if (nx == 0 || nrow_tiles == 0) return 0;
  Grid3 gr = make_grid(nx, nrow_tiles, B);
  const bool prof = gptq2d_prof_on(PROF_FLUSH);
  if (prof) gptq2d_prof_begin(PROF_FLUSH, stream);
  hipLaunchKernelGGL(flush_mfma_kernel<T>, gr.grid, dim3(256), 0, stream, y, c, e, l, u, g, lmap, umap, gr.nx, gr.ny);
  if (prof) gptq2d_prof_end(PROF_FLUSH, (double)B * gptq2d_flush_flops(m, n, P, Q, s0, s1, s_end), stream);
  return (int)hipGetLastError();
}

int gptq2d_flush_tiles_mfma_kron(float* y, float* c, const float* e, const float* l, const KronU& kr, int64_t m,
                                 int64_t n, int64_t S0, int64_t S1, int64_t S_end, hipStream_t stream);

// The fused sweep's flush with U = P (x) Q read from its factors (32 x 32 tiles, fp32, one matrix).
int gptq2d_flush_kron(float* y, float* c, const float* e, const float* l, const KronU& kr, int64_t m, int64_t n,
                      int64_t s0, int64_t s1, int64_t s_end, hipStream_t stream) {
  if (m <= 0 || n <= 0 || s0 < 0 || s1 <= s0 || s_end < s1) return GPTQ2D_EINVAL;
  if (s_end == s1) return 0;
  const bool prof = gptq2d_prof_on(PROF_FLUSH);
  if (prof) gptq2d_prof_begin(PROF_FLUSH, stream);
  const int rc = gptq2d_flush_tiles_mfma_kron(y, c, e, l, kr, m, n, s0, s1, s_end, stream);
  if (prof) gptq2d_prof_end(PROF_FLUSH, gptq2d_flush_flops(m, n, 32, 32, s0, s1, s_end), stream);
  return rc;
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
