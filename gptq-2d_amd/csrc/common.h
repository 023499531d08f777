// Shared device/host helpers for the GPTQ-2D HIP library (gfx950 only).
//
// Conventions used by every kernel in this library:
//  * Y, C and E are contiguous row-major [B, m, n] (B = product of the broadcast
//    batch shape).  The factors L [*, m, m] and U [*, n, n], and the quantizer
//    inputs, may broadcast over the batch: their element offset for logical batch
//    b comes from a BatchMap (shape of the broadcast batch and the operand's batch
//    strides, 0 on broadcast dimensions), passed by value so that a launch holds
//    no pointer to host memory and can be captured in a hipGraph.
//  * No kernel allocates, synchronises with the host or uses atomics, so every
//    entry point is deterministic and safe under stream capture.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define GPTQ2D_MAX_BATCH_DIMS 8

// Error codes returned by the C ABI besides hipError_t values (which are > 0).
#define GPTQ2D_EINVAL (-1)
#define GPTQ2D_EUNSUPPORTED (-2)
#define GPTQ2D_ESCRATCH (-3)

struct BatchMap {
  int32_t nd;
  int64_t shape[GPTQ2D_MAX_BATCH_DIMS];
  int64_t stride[GPTQ2D_MAX_BATCH_DIMS];

  // Element offset of logical batch b (row-major over shape, last dim fastest).
  __host__ __device__ __forceinline__ int64_t offset(int64_t b) const {
    int64_t off = 0;
    for (int d = nd - 1; d >= 0; --d) {
      const int64_t sz = shape[d];
      off += (b % sz) * stride[d];
      b /= sz;
    }
    return off;
  }
};

// Build a BatchMap from host arrays (nd <= GPTQ2D_MAX_BATCH_DIMS); returns false on bad input.
static inline bool make_batch_map(BatchMap& bm, int32_t nd, const int64_t* shape, const int64_t* stride) {
  if (nd < 0 || nd > GPTQ2D_MAX_BATCH_DIMS) return false;
  bm.nd = nd;
  for (int d = 0; d < GPTQ2D_MAX_BATCH_DIMS; ++d) {
    bm.shape[d] = d < nd ? shape[d] : 1;
    bm.stride[d] = (d < nd && stride) ? stride[d] : 0;
  }
  return true;
}

// U = P (x) Q given by its two factors, P [np, np] and Q [nq, nq] (row-major fp32, nq a multiple of 16), instead
// of its n^2 = (np nq)^2 entries:
//   U[i, j] = P[i / nq, j / nq] * Q[i % nq, j % nq],
// each entry formed by one fp32 multiplication, as torch.kron forms the explicit product (the same bits).  Since
// 16 divides nq, every aligned run of 16 rows or columns lies in one block of P: indices are split in units of
// 16, u = i / 16 = d16 (i / nq) + (i % nq) / 16 with d16 = nq / 16, by a multiply-high (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994): exact for every 32-bit dividend, and on the
// scalar unit for uniform ones.
struct KronU {
  const float* p;
  const float* q;
  int np, nq, d16;
  unsigned mag;  // floor(2^32 (2^l - d16) / d16) + 1, l = ceil(log2 d16)
  int sh1, sh2;  // min(l, 1), max(l - 1, 0)
};

static inline bool make_kron_u(KronU& k, const float* p, const float* q, int64_t np, int64_t nq) {
  if (!p || !q || np <= 0 || nq <= 0 || nq % 16 || np >= ((int64_t)1 << 26) || nq >= ((int64_t)1 << 26) ||
      np * nq >= ((int64_t)1 << 26))
    return false;
  k.p = p;
  k.q = q;
  k.np = (int)np;
  k.nq = (int)nq;
  k.d16 = (int)(nq / 16);
  int l = 0;
  while (((int64_t)1 << l) < k.d16) ++l;
  k.mag = (unsigned)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - (uint64_t)k.d16)) / (uint64_t)k.d16 + 1);
  k.sh1 = l < 1 ? l : 1;
  k.sh2 = l - 1 > 0 ? l - 1 : 0;
  return true;
}

// A 16-row (or column) unit u split as u = d16 i + r, 0 <= r < d16: index 16 u + w (0 <= w < 16) is row
// 16 r + w of block i of P.
__device__ __forceinline__ void kron_split(const KronU& k, unsigned u, int& i, int& r) {
  const unsigned t1 = __umulhi(k.mag, u);
  i = (int)((t1 + ((u - t1) >> k.sh1)) >> k.sh2);
  r = (int)u - i * k.d16;
}

// P[idx] for a wave-uniform idx, read through the scalar data cache (P is never written while a kernel reads it).
__device__ __forceinline__ float kron_p_uniform(const KronU& k, int idx) {
  typedef const __attribute__((address_space(4))) float* cptr;
  return ((cptr)k.p)[__builtin_amdgcn_readfirstlane(idx)];
}

// (block of P, index in Q) of index j of U's rows or columns.
__device__ __forceinline__ void kron_index(const KronU& k, int j, int& blk, int& in_q) {
  int r;
  kron_split(k, (unsigned)(j >> 4), blk, r);
  in_q = 16 * r + (j & 15);
}

static inline int64_t batch_count(int32_t nd, const int64_t* shape) {
  int64_t b = 1;
  for (int d = 0; d < nd; ++d) b *= shape[d];
  return b;
}

__host__ __device__ static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (queried once per device and host thread).
static inline int device_cus() {
  thread_local int cached_dev = -1, cached_cus = 256;
  int dev = 0;
  if (hipGetDevice(&dev) == hipSuccess && dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) {
      cached_cus = cus;
      cached_dev = dev;
    }
  }
  return cached_cus;
}

// Launch grid helper: (x, y, batch) as a 3-D grid while y and batch fit the
// 65535 limit of those axes, else every block linearised on axis x.  Kernels
// decode with GridIds.
struct Grid3 {
  dim3 grid;
  int64_t nx, ny;
};

static inline Grid3 make_grid(int64_t nx, int64_t ny, int64_t nb) {
  Grid3 g;
  g.nx = nx;
  g.ny = ny;
  if (ny <= 65535 && nb <= 65535) {
    g.grid = dim3((unsigned)nx, (unsigned)ny, (unsigned)nb);
  } else {
    g.grid = dim3((unsigned)(nx * ny * nb), 1, 1);
  }
  return g;
}

struct GridIds {
  int64_t x, y, b;
};

__device__ __forceinline__ GridIds grid_ids(int64_t nx, int64_t ny) {
  GridIds id;
  if ((int64_t)gridDim.x == nx) {
    id.x = blockIdx.x;
    id.y = blockIdx.y;
    id.b = blockIdx.z;
  } else {
    const int64_t lin = blockIdx.x;
    id.x = lin % nx;
    id.y = (lin / nx) % ny;
    id.b = lin / (nx * ny);
  }
  return id;
}

// Round half to even (IEEE rint); matches torch.round.
__device__ __forceinline__ float round_even(float x) { return __builtin_rintf(x); }
__device__ __forceinline__ double round_even(double x) { return __builtin_rint(x); }

template <typename T>
__device__ __forceinline__ T clamp_val(T x, T lo, T hi) {
  // NaN propagates like torch.clamp: comparisons with NaN are false.
  x = x < lo ? lo : x;
  x = x > hi ? hi : x;
  return x;
}

// fp32 -> bf16 / fp16 with round-to-nearest-even, returned as fp32.  Written
// from the IEEE-754 definitions (bit manipulation), NaN kept quiet.
__device__ __forceinline__ float round_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return __uint_as_float(u | 0x00400000u);  // NaN
  const uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return __uint_as_float(u & 0xffff0000u);
}

__device__ __forceinline__ float round_to_fp16(float f) {
  // The hardware conversion v_cvt_f16_f32 rounds to nearest even and keeps denormals.
  return (float)(_Float16)f;
}

template <typename T>
__device__ __forceinline__ T round_scale16(T s, int dtype16) {
  const float f = (float)s;  // as PyTorch: to fp32, then to the 16-bit dtype
  const float r = dtype16 == 1 ? round_to_bf16(f) : round_to_fp16(f);
  return (T)r;
}
