// Per-stage kernels of the plug-in path of the GPTQ-2D sweep.
//
// When the quantizer is an arbitrary Python callable, the host calls it once per
// antidiagonal (stage) and these kernels apply that stage's error feedback inside
// the current block of stages.  The block's feedback into later stages is applied
// by the flush kernel (flush.hip).  Every kernel owns its output elements, so there
// are no atomics and results are deterministic.
//
// Reference counterparts (IST-DASLab/GPTQ-2D, gptq_2d.py):
//   push_plain_kernel     <- _push_kernel                     :244-346
//   add_own_errors_kernel <- _add_own_errors_kernel           :382-409
//   push_down_se_kernel   <- _push_down_super_entry_kernel    :429-505
//   push_right_se_kernel  <- _push_right_super_entry_kernel   :537-601
//   gather_kernel         <- the old-value copy in _gptq_2d_blocked :1345-1348
#include "common.h"

namespace {

// ------------------------------------------------------------------------------------------------
// Plain entries.  Stage s holds sources (i, s-i) for rows lo <= i < hi; lane k = i - lo of z and
// old.  A thread owns one receiver (r, s-r+p): p = 0 commits the source of row r; 1 <= p <= reach
// receives the down push of source (r-p, s-r+p) and the right push of source (r, s-r).  The error
// of a source is z - old, where old holds Y on the stage before quantisation (the p = 1 receivers
// of the previous stage, saved by that stage's launch), so committing z never races a reader.
// C at the sources is left untouched here; add_own_errors folds the errors in after the block.
template <typename T>
__global__ __launch_bounds__(256) void push_plain_kernel(T* __restrict__ y, T* __restrict__ c, T* __restrict__ e,
                                                         const T* __restrict__ z, const T* __restrict__ old,
                                                         T* __restrict__ next_old, const T* __restrict__ l,
                                                         const T* __restrict__ u, int64_t m, int64_t n, int64_t s,
                                                         int64_t reach, int64_t nrows, BatchMap lmap, BatchMap umap,
                                                         int64_t nx, int64_t ny) {
  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t lo = s - n + 1 > 0 ? s - n + 1 : 0;
  const int64_t hi = s + 1 < m ? s + 1 : m;
  const int64_t len = hi - lo;
  const int64_t lo1 = s - n + 2 > 0 ? s - n + 2 : 0;
  const int64_t len1 = (s + 2 < m ? s + 2 : m) - lo1;
  const int64_t r = lo + id.x * 8 + (threadIdx.x >> 5);
  if (r - lo >= nrows || r >= m) return;
  const T* zb = z + b * len;
  const T* ob = old + b * len;
  const int64_t mat = b * m * n;
  const bool has_src = r < hi;
  for (int64_t p = (threadIdx.x & 31) + id.y * 32; p <= reach; p += 32 * ny) {
    if (p == 0) {
      if (has_src) {
        const T zr = zb[r - lo];
        y[mat + r * n + (s - r)] = zr;
        e[mat + r * n + (s - r)] = zr - ob[r - lo];
      }
      continue;
    }
    const int64_t j = s - r + p;
    if (j >= n) continue;
    const int64_t i = r - p;  // row of the source pushing down into (r, j)
    const bool down_ok = i >= lo && i < hi;
    const bool right_ok = has_src;
    if (!down_ok && !right_ok) continue;
    const int64_t off = mat + r * n + j;
    T yv = y[off];
    if (down_ok) {
      const T err = zb[i - lo] - ob[i - lo];
      const T dv = l[lmap.offset(b) + r * m + i] * err;
      c[off] = c[off] + dv;
      yv = yv + dv;
    }
    if (right_ok) {
      const T own_c = c[mat + r * n + (s - r)] + (zb[r - lo] - ob[r - lo]);
      yv = yv + own_c * u[umap.offset(b) + (s - r) * n + j];
    }
    y[off] = yv;
    if (p == 1) next_old[b * len1 + (r - lo1)] = yv;  // final: Y on the next stage before quantisation
  }
}

// C[r, s-r] += E[r, s-r] for the stages s0 <= s < s1 of a finished block.
template <typename T>
__global__ __launch_bounds__(256) void add_own_errors_kernel(T* __restrict__ c, const T* __restrict__ e, int64_t m,
                                                             int64_t n, int64_t s0, int64_t s1, int64_t row0,
                                                             int64_t nx, int64_t ny) {
  const GridIds id = grid_ids(nx, ny);
  const int64_t r = row0 + id.x * 8 + (threadIdx.x >> 5);
  const int64_t d = id.y * 32 + (threadIdx.x & 31);
  const int64_t s = s0 + d;
  if (r >= m || s >= s1) return;
  const int64_t j = s - r;
  if (j < 0 || j >= n) return;
  const int64_t off = id.b * m * n + r * n + j;
  c[off] = c[off] + e[off];
}

// ------------------------------------------------------------------------------------------------
// Super-entries p x q.  Source lane k of coarse stage s is super-entry (ib, jb) = (lo+k, s-lo-k).
// Down: every row r of [ib*p, rows_end) receives C[r, jb band] += L[r, ib band] E, the super-entry's
// own rows through the implicit identity block (which folds E into C), and rows below it the same
// update in Y.  Sources own distinct column bands, so blocks never share an output.
template <typename T>
__global__ __launch_bounds__(256) void push_down_se_kernel(T* __restrict__ y, T* __restrict__ c, T* __restrict__ e,
                                                           const T* __restrict__ z, const T* __restrict__ l,
                                                           int64_t m, int64_t n, int64_t p, int64_t q, int64_t s,
                                                           int64_t s1, int64_t rows_per_block, BatchMap lmap,
                                                           int64_t nx, int64_t ny) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* err = reinterpret_cast<T*>(smem_raw);  // [p][q]
  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t lo = s - n / q + 1 > 0 ? s - n / q + 1 : 0;
  const int64_t len = (s + 1 < m / p ? s + 1 : m / p) - lo;
  const int64_t k = id.x;
  const int64_t ib = lo + k, jb = s - ib;
  const int64_t rows_end = (s1 - jb) * p < m ? (s1 - jb) * p : m;
  const int64_t r0 = ib * p + id.y * rows_per_block;
  if (r0 >= rows_end) return;
  const int64_t mat = b * m * n;
  const T* zk = z + (b * len + k) * p * q;
  for (int64_t t = threadIdx.x; t < p * q; t += blockDim.x) {
    const int64_t a = t / q, bq = t % q;
    const int64_t src = mat + (ib * p + a) * n + jb * q + bq;
    const T ev = zk[t] - y[src];
    err[t] = ev;
    if (id.y == 0) e[src] = ev;
  }
  __syncthreads();
  const T* lb = l + lmap.offset(b);
  const int64_t r1 = r0 + rows_per_block < rows_end ? r0 + rows_per_block : rows_end;
  for (int64_t t = threadIdx.x; t < (r1 - r0) * q; t += blockDim.x) {
    const int64_t r = r0 + t / q, bq = t % q;
    const int64_t off = mat + r * n + jb * q + bq;
    if (r < ib * p + p) {
      c[off] = c[off] + err[(r - ib * p) * q + bq];
    } else {
      T acc = 0;
      const T* lr = lb + r * m + ib * p;
      for (int64_t a = 0; a < p; ++a) acc += lr[a] * err[a * q + bq];
      c[off] = c[off] + acc;
      y[off] = y[off] + acc;
    }
  }
}

// Right: commit z into the super-entry, then every column c of [(jb+1)*q, cols_end) in its row band
// receives Y[ib band, c] += C[ib band, jb band] U[jb band, c].  Runs after push_down_se (C complete).
template <typename T>
__global__ __launch_bounds__(256) void push_right_se_kernel(T* __restrict__ y, const T* __restrict__ c,
                                                            const T* __restrict__ z, const T* __restrict__ u,
                                                            int64_t m, int64_t n, int64_t p, int64_t q, int64_t s,
                                                            int64_t s1, int64_t cols_per_block, BatchMap umap,
                                                            int64_t nx, int64_t ny) {
  extern __shared__ __align__(16) unsigned char smem_raw[];
  T* cs = reinterpret_cast<T*>(smem_raw);  // [p][q]
  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t lo = s - n / q + 1 > 0 ? s - n / q + 1 : 0;
  const int64_t len = (s + 1 < m / p ? s + 1 : m / p) - lo;
  const int64_t k = id.x;
  const int64_t ib = lo + k, jb = s - ib;
  const int64_t mat = b * m * n;
  if (id.y == 0) {
    const T* zk = z + (b * len + k) * p * q;
    for (int64_t t = threadIdx.x; t < p * q; t += blockDim.x)
      y[mat + (ib * p + t / q) * n + jb * q + t % q] = zk[t];
  }
  const int64_t cols_end = (s1 - ib) * q < n ? (s1 - ib) * q : n;
  const int64_t c0 = (jb + 1) * q + id.y * cols_per_block;
  if (c0 >= cols_end) return;
  for (int64_t t = threadIdx.x; t < p * q; t += blockDim.x)
    cs[t] = c[mat + (ib * p + t / q) * n + jb * q + t % q];
  __syncthreads();
  const T* ub = u + umap.offset(b);
  const int64_t c1 = c0 + cols_per_block < cols_end ? c0 + cols_per_block : cols_end;
  const int64_t w = c1 - c0;
  for (int64_t t = threadIdx.x; t < p * w; t += blockDim.x) {
    const int64_t a = t / w, col = c0 + t % w;
    T acc = 0;
    for (int64_t bq = 0; bq < q; ++bq) acc += cs[a * q + bq] * ub[(jb * q + bq) * n + col];
    const int64_t off = mat + (ib * p + a) * n + col;
    y[off] = y[off] + acc;
  }
}

// out[b, k] = Y[b, lo+k, s-lo-k]: the antidiagonal's values before its first push in a block.
template <typename T>
__global__ __launch_bounds__(256) void gather_kernel(const T* __restrict__ y, T* __restrict__ out, int64_t m,
                                                     int64_t n, int64_t s, int64_t len, int64_t nb) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= len * nb) return;
  const int64_t b = t / len, k = t % len;
  const int64_t lo = s - n + 1 > 0 ? s - n + 1 : 0;
  out[t] = y[b * m * n + (lo + k) * n + (s - lo - k)];
}

template <typename T>
__global__ void fill_kernel(T* __restrict__ x, T v, int64_t count) {
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < count; t += (int64_t)gridDim.x * blockDim.x)
    x[t] = v;
}

// ------------------------------------------------------------------------------------------------ host side

template <typename T>
int push_plain(T* y, T* c, T* e, const T* z, const T* old, T* next_old, const T* l, const T* u, int64_t m, int64_t n,
               int64_t s, int64_t s1, int32_t bnd, const int64_t* bshape, const int64_t* lstride,
               const int64_t* ustride, hipStream_t stream) {
  BatchMap lmap, umap;
  if (!make_batch_map(lmap, bnd, bshape, lstride) || !make_batch_map(umap, bnd, bshape, ustride)) return GPTQ2D_EINVAL;
  if (m <= 0 || n <= 0 || s < 0 || s > m + n - 2 || s1 <= s) return GPTQ2D_EINVAL;
  const int64_t B = batch_count(bnd, bshape);
  if (B == 0) return 0;
  const int64_t lo = s - n + 1 > 0 ? s - n + 1 : 0;
  const int64_t hi = s + 1 < m ? s + 1 : m;
  const int64_t reach = s1 - s - 1;
  const int64_t last = hi - 1 + reach + 1 < m ? hi - 1 + reach + 1 : m;  // one past the last receiver row
  const int64_t nrows = last - lo;
  const int64_t ny = cdiv(reach + 1, 32) < 4 ? cdiv(reach + 1, 32) : 4;
  Grid3 g = make_grid(cdiv(nrows, 8), ny, B);
  hipLaunchKernelGGL(push_plain_kernel<T>, g.grid, dim3(256), 0, stream, y, c, e, z, old, next_old, l, u, m, n, s,
                     reach, nrows, lmap, umap, g.nx, g.ny);
  return (int)hipGetLastError();
}

template <typename T>
int add_own_errors(T* c, const T* e, int64_t B, int64_t m, int64_t n, int64_t s0, int64_t s1, hipStream_t stream) {
  if (m <= 0 || n <= 0 || s1 <= s0 || B < 0) return GPTQ2D_EINVAL;
  if (B == 0) return 0;
  const int64_t row0 = s0 - n + 1 > 0 ? s0 - n + 1 : 0;
  const int64_t row1 = s1 < m ? s1 : m;
  if (row1 <= row0) return 0;
  Grid3 g = make_grid(cdiv(row1 - row0, 8), cdiv(s1 - s0, 32), B);
  hipLaunchKernelGGL(add_own_errors_kernel<T>, g.grid, dim3(256), 0, stream, c, e, m, n, s0, s1, row0, g.nx, g.ny);
  return (int)hipGetLastError();
}

template <typename T>
int push_down_se(T* y, T* c, T* e, const T* z, const T* l, int64_t m, int64_t n, int64_t p, int64_t q, int64_t s,
                 int64_t s1, int32_t bnd, const int64_t* bshape, const int64_t* lstride, hipStream_t stream) {
  BatchMap lmap;
  if (!make_batch_map(lmap, bnd, bshape, lstride)) return GPTQ2D_EINVAL;
  if (p <= 0 || q <= 0 || m % p || n % q || s1 <= s) return GPTQ2D_EINVAL;
  if ((int64_t)sizeof(T) * p * q > 64 * 1024) return GPTQ2D_EUNSUPPORTED;
  const int64_t B = batch_count(bnd, bshape);
  if (B == 0) return 0;
  const int64_t lo = s - n / q + 1 > 0 ? s - n / q + 1 : 0;
  const int64_t hi = s + 1 < m / p ? s + 1 : m / p;
  const int64_t rows = (m - lo * p) < (s1 - s) * p ? (m - lo * p) : (s1 - s) * p;  // longest push: first source
  const int64_t rows_per_block = 64;
  Grid3 g = make_grid(hi - lo, cdiv(rows, rows_per_block), B);
  hipLaunchKernelGGL(push_down_se_kernel<T>, g.grid, dim3(256), sizeof(T) * p * q, stream, y, c, e, z, l, m, n, p, q,
                     s, s1, rows_per_block, lmap, g.nx, g.ny);
  return (int)hipGetLastError();
}

template <typename T>
int push_right_se(T* y, const T* c, const T* z, const T* u, int64_t m, int64_t n, int64_t p, int64_t q, int64_t s,
                  int64_t s1, int32_t bnd, const int64_t* bshape, const int64_t* ustride, hipStream_t stream) {
  BatchMap umap;
  if (!make_batch_map(umap, bnd, bshape, ustride)) return GPTQ2D_EINVAL;
  if (p <= 0 || q <= 0 || m % p || n % q || s1 <= s) return GPTQ2D_EINVAL;
  if ((int64_t)sizeof(T) * p * q > 64 * 1024) return GPTQ2D_EUNSUPPORTED;
  const int64_t B = batch_count(bnd, bshape);
  if (B == 0) return 0;
  const int64_t lo = s - n / q + 1 > 0 ? s - n / q + 1 : 0;
  const int64_t hi = s + 1 < m / p ? s + 1 : m / p;
  const int64_t jlo = s - (hi - 1);  // the last source pushes farthest right
  const int64_t cols_a = n - (jlo + 1) * q, cols_b = (s1 - s - 1) * q;
  const int64_t cols = cols_a < cols_b ? cols_a : cols_b;
  const int64_t cols_per_block = 256;
  const int64_t ny = cols > 0 ? cdiv(cols, cols_per_block) : 1;  // at least one block commits z
  Grid3 g = make_grid(hi - lo, ny, B);
  hipLaunchKernelGGL(push_right_se_kernel<T>, g.grid, dim3(256), sizeof(T) * p * q, stream, y, c, z, u, m, n, p, q, s,
                     s1, cols_per_block, umap, g.nx, g.ny);
  return (int)hipGetLastError();
}

template <typename T>
int gather(const T* y, T* out, int64_t B, int64_t m, int64_t n, int64_t s, hipStream_t stream) {
  if (m <= 0 || n <= 0 || s < 0 || s > m + n - 2) return GPTQ2D_EINVAL;
  const int64_t lo = s - n + 1 > 0 ? s - n + 1 : 0;
  const int64_t len = (s + 1 < m ? s + 1 : m) - lo;
  if (B * len == 0) return 0;
  hipLaunchKernelGGL(gather_kernel<T>, dim3((unsigned)cdiv(B * len, 256)), dim3(256), 0, stream, y, out, m, n, s, len,
                     B);
  return (int)hipGetLastError();
}

}  // namespace

template <typename T>
int gptq2d_fill(T* x, T v, int64_t count, hipStream_t stream) {
  if (count <= 0) return count < 0 ? GPTQ2D_EINVAL : 0;
  const int64_t blocks = cdiv(count, 256) < 4096 ? cdiv(count, 256) : 4096;
  hipLaunchKernelGGL(fill_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, x, v, count);
  return (int)hipGetLastError();
}
template int gptq2d_fill<float>(float*, float, int64_t, hipStream_t);
template int gptq2d_fill<double>(double*, double, int64_t, hipStream_t);

extern "C" {

#define GPTQ2D_GENERIC_ABI(SUF, T)                                                                                   \
  int gptq2d_push_plain_##SUF(T* y, T* c, T* e, const T* z, const T* old, T* next_old, const T* l, const T* u,     \
                              int64_t m, int64_t n, int64_t s, int64_t s1, int32_t bnd, const int64_t* bshape,    \
                              const int64_t* lstride, const int64_t* ustride, hipStream_t stream) {                \
    return push_plain<T>(y, c, e, z, old, next_old, l, u, m, n, s, s1, bnd, bshape, lstride, ustride, stream);     \
  }                                                                                                                  \
  int gptq2d_add_own_errors_##SUF(T* c, const T* e, int64_t B, int64_t m, int64_t n, int64_t s0, int64_t s1,        \
                                  hipStream_t stream) {                                                             \
    return add_own_errors<T>(c, e, B, m, n, s0, s1, stream);                                                         \
  }                                                                                                                  \
  int gptq2d_push_down_se_##SUF(T* y, T* c, T* e, const T* z, const T* l, int64_t m, int64_t n, int64_t p,          \
                                int64_t q, int64_t s, int64_t s1, int32_t bnd, const int64_t* bshape,               \
                                const int64_t* lstride, hipStream_t stream) {                                       \
    return push_down_se<T>(y, c, e, z, l, m, n, p, q, s, s1, bnd, bshape, lstride, stream);                          \
  }                                                                                                                  \
  int gptq2d_push_right_se_##SUF(T* y, const T* c, const T* z, const T* u, int64_t m, int64_t n, int64_t p,         \
                                 int64_t q, int64_t s, int64_t s1, int32_t bnd, const int64_t* bshape,              \
                                 const int64_t* ustride, hipStream_t stream) {                                      \
    return push_right_se<T>(y, c, z, u, m, n, p, q, s, s1, bnd, bshape, ustride, stream);                            \
  }                                                                                                                  \
  int gptq2d_gather_antidiagonal_##SUF(const T* y, T* out, int64_t B, int64_t m, int64_t n, int64_t s,              \
                                       hipStream_t stream) {                                                        \
    return gather<T>(y, out, B, m, n, s, stream);                                                                    \
  }                                                                                                                  \
  int gptq2d_fill_##SUF(T* x, double v, int64_t count, hipStream_t stream) {                                        \
    return gptq2d_fill<T>(x, (T)v, count, stream);                                                                   \
  }

GPTQ2D_GENERIC_ABI(f32, float)
GPTQ2D_GENERIC_ABI(f64, double)

}  // extern "C"
