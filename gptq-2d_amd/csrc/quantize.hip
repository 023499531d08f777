// Quantizer plug-in kernels: one launch quantizes and dequantizes the selected entries of one
// antidiagonal (a flat strided slice) or of its super-entries (a strided [d, p, q] view).
//
// Numerics (reference quantizer_int.py): correctly rounded division (hipcc's default IEEE fp32
// divide), round half to even (rint), denormals preserved, and the 16-bit scale rounding from
// fp32 with round-to-nearest-even.
//   affine_slice_kernel <- _affine_quantize_kernel              quantizer_int.py:161-205
//   affine_se_kernel    <- _affine_quantize_super_entry_kernel  quantizer_int.py:248-299
//   absmax_scale_kernel <- _int_abs_max_scale_kernel            quantizer_int.py:358-385
//   absmax_se_kernel    <- _int_abs_max_quantize_kernel         quantizer_int.py:408-439
//   round kernels       <- round_quantizer(_super_entry) (torch.round)  quantizer_int.py:18-35
#include "common.h"

namespace {

template <typename T>
__device__ __forceinline__ T affine_q(T y, T s, T z, T qmin, T qmax) {
  const T code = clamp_val(round_even(y / s + z), qmin, qmax);
  return (code - z) * s;
}

// Entry k of the slice sits at flat position start + k*step of every matrix-shaped operand.
template <typename T, bool AFFINE>
__global__ __launch_bounds__(256) void slice_kernel(T* __restrict__ out, const T* __restrict__ y,
                                                    const T* __restrict__ scale, const T* __restrict__ zp,
                                                    int64_t msize, int64_t start, int64_t step, int64_t len,
                                                    BatchMap smap, BatchMap zmap, T qmin, T qmax, int64_t nx,
                                                    int64_t ny) {
  const GridIds id = grid_ids(nx, ny);
  const int64_t k = id.x * 256 + threadIdx.x;
  if (k >= len) return;
  const int64_t b = id.b;
  const int64_t pos = start + k * step;
  const T yv = y[b * msize + pos];
  T z;
  if (AFFINE)
    z = affine_q(yv, scale[smap.offset(b) + pos], zp[zmap.offset(b) + pos], qmin, qmax);
  else
    z = round_even(yv);
  out[b * len + k] = z;
}

// Super-entry e = (kk, r, c) of the view sits kk*sd + r*sp + c*sq past each operand's first
// selected entry; out is the contiguous [B, d, p, q].
template <typename T, bool AFFINE>
__global__ __launch_bounds__(256) void se_kernel(T* __restrict__ out, const T* __restrict__ y,
                                                 const T* __restrict__ scale, const T* __restrict__ zp,
                                                 int64_t msize, int64_t d, int64_t p, int64_t q, int64_t sd,
                                                 int64_t sp, int64_t sq, BatchMap smap, BatchMap zmap, T qmin, T qmax,
                                                 int64_t nx, int64_t ny) {
  const GridIds id = grid_ids(nx, ny);
  const int64_t len = d * p * q;
  const int64_t t = id.x * 256 + threadIdx.x;
  if (t >= len) return;
  const int64_t b = id.b;
  const int64_t kk = t / (p * q), r = (t / q) % p, cc = t % q;
  const int64_t pos = kk * sd + r * sp + cc * sq;
  const T yv = y[b * msize + pos];
  T z;
  if (AFFINE)
    z = affine_q(yv, scale[smap.offset(b) + pos], zp[zmap.offset(b) + pos], qmin, qmax);
  else
    z = round_even(yv);
  out[b * len + t] = z;
}

// absmax / (range/2), rounded to the 16-bit dtype through fp32, zero -> 1.
template <typename T>
__device__ __forceinline__ T absmax_scale(T amax, T half_range, int dtype16) {
  T s = amax / half_range;
  s = round_scale16(s, dtype16);
  return s == T(0) ? T(1) : s;
}

template <typename T>
__global__ __launch_bounds__(256) void absmax_scale_kernel(T* __restrict__ out, const T* __restrict__ x,
                                                           int64_t rows, int64_t size, int64_t rs, int64_t cs,
                                                           T half_range, int dtype16) {
  const int64_t row = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (row >= rows) return;
  T amax = T(0);
  for (int64_t k = 0; k < size; ++k) {
    const T a = fabs(x[row * rs + k * cs]);
    amax = a > amax ? a : amax;
  }
  out[row] = absmax_scale(amax, half_range, dtype16);
}

// One thread per row of one super-entry: scale from the row's current abs max, then
// clamp(rint(y / s), qmin, qmax) * s.  scale_out (optional): a per-entry map laid out like y (the same view
// strides), where every entry of the row receives the row's scale.
template <typename T>
__global__ __launch_bounds__(256) void absmax_se_kernel(T* __restrict__ out, const T* __restrict__ y, int64_t msize,
                                                        int64_t d, int64_t p, int64_t q, int64_t sd, int64_t sp,
                                                        int64_t sq, T qmin, T qmax, int dtype16,
                                                        T* __restrict__ scale_out, int64_t nx, int64_t ny) {
  const GridIds id = grid_ids(nx, ny);
  const int64_t rr = id.x * 256 + threadIdx.x;
  if (rr >= d * p) return;
  const int64_t b = id.b;
  const int64_t kk = rr / p, r = rr % p;
  const T* yr = y + b * msize + kk * sd + r * sp;
  T amax = T(0);
  for (int64_t cc = 0; cc < q; ++cc) {
    const T a = fabs(yr[cc * sq]);
    amax = a > amax ? a : amax;
  }
  const T s = absmax_scale(amax, (qmax - qmin) / T(2), dtype16);
  T* o = out + (b * d * p + rr) * q;
  for (int64_t cc = 0; cc < q; ++cc) o[cc] = clamp_val(round_even(yr[cc * sq] / s), qmin, qmax) * s;
  if (scale_out) {
    T* so = scale_out + b * msize + kk * sd + r * sp;
    for (int64_t cc = 0; cc < q; ++cc) so[cc * sq] = s;
  }
}

template <typename T>
int slice_quantize(bool affine, T* out, const T* y, const T* scale, const T* zp, int64_t msize, int64_t start,
                   int64_t step, int64_t len, int32_t bnd, const int64_t* bshape, const int64_t* sstride,
                   const int64_t* zstride, double qmin, double qmax, hipStream_t stream) {
  BatchMap smap, zmap;
  if (!make_batch_map(smap, bnd, bshape, sstride) || !make_batch_map(zmap, bnd, bshape, zstride)) return GPTQ2D_EINVAL;
  if (len < 0 || (affine && (!scale || !zp))) return GPTQ2D_EINVAL;
  const int64_t B = batch_count(bnd, bshape);
  if (B == 0 || len == 0) return 0;
  Grid3 g = make_grid(cdiv(len, 256), 1, B);
  if (affine)
    hipLaunchKernelGGL((slice_kernel<T, true>), g.grid, dim3(256), 0, stream, out, y, scale, zp, msize, start, step,
                       len, smap, zmap, (T)qmin, (T)qmax, g.nx, g.ny);
  else
    hipLaunchKernelGGL((slice_kernel<T, false>), g.grid, dim3(256), 0, stream, out, y, scale, zp, msize, start, step,
                       len, smap, zmap, (T)qmin, (T)qmax, g.nx, g.ny);
  return (int)hipGetLastError();
}

template <typename T>
int se_quantize(bool affine, T* out, const T* y, const T* scale, const T* zp, int64_t msize, int64_t d, int64_t p,
                int64_t q, int64_t sd, int64_t sp, int64_t sq, int32_t bnd, const int64_t* bshape,
                const int64_t* sstride, const int64_t* zstride, double qmin, double qmax, hipStream_t stream) {
  BatchMap smap, zmap;
  if (!make_batch_map(smap, bnd, bshape, sstride) || !make_batch_map(zmap, bnd, bshape, zstride)) return GPTQ2D_EINVAL;
  if (d < 0 || p <= 0 || q <= 0 || (affine && (!scale || !zp))) return GPTQ2D_EINVAL;
  const int64_t B = batch_count(bnd, bshape);
  if (B == 0 || d == 0) return 0;
  Grid3 g = make_grid(cdiv(d * p * q, 256), 1, B);
  if (affine)
    hipLaunchKernelGGL((se_kernel<T, true>), g.grid, dim3(256), 0, stream, out, y, scale, zp, msize, d, p, q, sd, sp,
                       sq, smap, zmap, (T)qmin, (T)qmax, g.nx, g.ny);
  else
    hipLaunchKernelGGL((se_kernel<T, false>), g.grid, dim3(256), 0, stream, out, y, scale, zp, msize, d, p, q, sd, sp,
                       sq, smap, zmap, (T)qmin, (T)qmax, g.nx, g.ny);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

#define GPTQ2D_QUANT_ABI(SUF, T)                                                                                     \
  int gptq2d_affine_quantize_##SUF(T* out, const T* y, const T* scale, const T* zp, int64_t msize, int64_t start,    \
                                   int64_t step, int64_t len, int32_t bnd, const int64_t* bshape,                    \
                                   const int64_t* sstride, const int64_t* zstride, double qmin, double qmax,         \
                                   hipStream_t stream) {                                                             \
    return slice_quantize<T>(true, out, y, scale, zp, msize, start, step, len, bnd, bshape, sstride, zstride, qmin,  \
                             qmax, stream);                                                                          \
  }                                                                                                                   \
  int gptq2d_round_quantize_##SUF(T* out, const T* y, int64_t msize, int64_t start, int64_t step, int64_t len,      \
                                  int32_t bnd, const int64_t* bshape, hipStream_t stream) {                          \
    return slice_quantize<T>(false, out, y, nullptr, nullptr, msize, start, step, len, bnd, bshape, nullptr,         \
                             nullptr, 0., 0., stream);                                                               \
  }                                                                                                                   \
  int gptq2d_affine_quantize_se_##SUF(T* out, const T* y, const T* scale, const T* zp, int64_t msize, int64_t d,     \
                                      int64_t p, int64_t q, int64_t sd, int64_t sp, int64_t sq, int32_t bnd,         \
                                      const int64_t* bshape, const int64_t* sstride, const int64_t* zstride,         \
                                      double qmin, double qmax, hipStream_t stream) {                                \
    return se_quantize<T>(true, out, y, scale, zp, msize, d, p, q, sd, sp, sq, bnd, bshape, sstride, zstride, qmin,  \
                          qmax, stream);                                                                             \
  }                                                                                                                   \
  int gptq2d_round_quantize_se_##SUF(T* out, const T* y, int64_t msize, int64_t d, int64_t p, int64_t q, int64_t sd, \
                                     int64_t sp, int64_t sq, int32_t bnd, const int64_t* bshape,                     \
                                     hipStream_t stream) {                                                           \
    return se_quantize<T>(false, out, y, nullptr, nullptr, msize, d, p, q, sd, sp, sq, bnd, bshape, nullptr,         \
                          nullptr, 0., 0., stream);                                                                  \
  }                                                                                                                   \
  int gptq2d_absmax_scale_##SUF(T* out, const T* x, int64_t rows, int64_t size, int64_t row_stride,                 \
                                int64_t col_stride, double qmin, double qmax, int32_t dtype16, hipStream_t stream) { \
    if (rows < 0 || size < 0 || !(qmin < qmax) || (dtype16 != 1 && dtype16 != 2)) return GPTQ2D_EINVAL;             \
    if (rows == 0) return 0;                                                                                          \
    hipLaunchKernelGGL(absmax_scale_kernel<T>, dim3((unsigned)cdiv(rows, 256)), dim3(256), 0, stream, out, x, rows,  \
                       size, row_stride, col_stride, (T)((qmax - qmin) / 2), dtype16);                               \
    return (int)hipGetLastError();                                                                                    \
  }                                                                                                                   \
  int gptq2d_absmax_quantize_se_##SUF(T* out, const T* y, int64_t msize, int64_t B, int64_t d, int64_t p, int64_t q, \
                                      int64_t sd, int64_t sp, int64_t sq, double qmin, double qmax, int32_t dtype16, \
                                      T* scale_out, hipStream_t stream) {                                            \
    if (B < 0 || d < 0 || p <= 0 || q <= 0 || !(qmin < qmax) || (dtype16 != 1 && dtype16 != 2))                     \
      return GPTQ2D_EINVAL;                                                                                           \
    if (B == 0 || d == 0) return 0;                                                                                   \
    Grid3 g = make_grid(cdiv(d * p, 256), 1, B);                                                                     \
    hipLaunchKernelGGL(absmax_se_kernel<T>, g.grid, dim3(256), 0, stream, out, y, msize, d, p, q, sd, sp, sq,        \
                       (T)qmin, (T)qmax, dtype16, scale_out, g.nx, g.ny);                                            \
    return (int)hipGetLastError();                                                                                    \
  }

GPTQ2D_QUANT_ABI(f32, float)
GPTQ2D_QUANT_ABI(f64, double)

}  // extern "C"
