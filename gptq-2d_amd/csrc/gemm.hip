// Strided batched GEMM with triangular operand structure, for the LDL preprocessing.
//
// D = beta D + alpha A B over arbitrary element strides, so the callers express transposes,
// reversals (negative strides) and sub-blocks without copies.  Structurally zero parts of
// triangular operands are skipped in the K loop and masked (at load time, or in LDS after an
// LDS-direct load), so they never reach the result.  fp32 runs on the MFMA path
// (v_mfma_f32_32x32x2_f32: 128 x 128 output tile per workgroup, four waves of 64 x 64, K staged
// through LDS 16 deep), fp32 products of fewer than 64 rows or columns on the VALU path (64 x 64 tile,
// 4 x 4 outputs per thread); fp64 on MFMA (v_mfma_f64_16x16x4_f64, 64 x 64 tile), with LDS-direct
// double-buffered panels where the operands' rows (A) and rows or columns (B) are contiguous.
#include "linalg.h"
#include "lds_dma.h"

namespace {

// ------------------------------------------------------------------------------------------------ shared

struct TileRange {
  int64_t k_lo, k_hi;
  bool empty;
};

template <typename T>
__device__ __forceinline__ TileRange tile_k_range(const GemmProblem<T>& p, int64_t i0, int64_t i1, int64_t j0,
                                                  int64_t j1) {
  TileRange r{0, p.K, false};
  if (p.a_tri == TRI_LOWER && i1 < r.k_hi) r.k_hi = i1;  // A(i,k) = 0 for k > i
  if (p.a_tri == TRI_UPPER && i0 > r.k_lo) r.k_lo = i0;  // A(i,k) = 0 for k < i
  if (p.b_tri == TRI_LOWER && j0 > r.k_lo) r.k_lo = j0;  // B(k,j) = 0 for k < j
  if (p.b_tri == TRI_UPPER && j1 < r.k_hi) r.k_hi = j1;  // B(k,j) = 0 for k > j
  if (p.d_tri == TRI_LOWER && j0 > i1 - 1) r.empty = true;
  if (p.d_tri == TRI_UPPER && i0 > j1 - 1) r.empty = true;
  return r;
}

template <typename T>
__device__ __forceinline__ T load_a(const GemmProblem<T>& p, const T* a, int64_t i, int64_t k, int64_t k_hi) {
  if (i >= p.M || k >= k_hi || k < 0) return T(0);
  if (p.a_tri == TRI_LOWER && k > i) return T(0);
  if (p.a_tri == TRI_UPPER && k < i) return T(0);
  return a[i * p.a_rs + k * p.a_cs];
}

template <typename T>
__device__ __forceinline__ T load_b(const GemmProblem<T>& p, const T* b, int64_t k, int64_t j, int64_t k_hi) {
  if (j >= p.N || k >= k_hi || k < 0) return T(0);
  if (p.b_tri == TRI_LOWER && k < j) return T(0);
  if (p.b_tri == TRI_UPPER && k > j) return T(0);
  return b[k * p.b_rs + j * p.b_cs];
}

// D = beta D + alpha acc for NV outputs of one lane, output x at (i, j) = at(x): every load of D first, then
// every new value (outside the stores' branches, so that one wait covers all loads), then the stores.
// Output by output (load, wait, store), the compiler must keep each load behind the previous store --
// through one pointer with run-time strides it cannot prove two outputs distinct -- and a tile's epilogue
// waited on one memory round trip per output (16 to 64 in a row).  Same arithmetic as one output at a
// time; D is not read where beta = 0.
template <int NV, typename T, typename At>
__device__ __forceinline__ void store_d_group(const GemmProblem<T>& p, T* d, const T (&acc)[NV], At at) {
  static_assert(NV <= 64, "one mask bit per output");
  T old[NV];
  uint64_t ok = 0;
#pragma unroll
  for (int x = 0; x < NV; ++x) {
    int64_t i, j;
    at(x, i, j);
    const bool in = i < p.M && j < p.N && !(p.d_tri == TRI_LOWER && j > i) && !(p.d_tri == TRI_UPPER && j < i);
    old[x] = T(0);
    if (in) {
      ok |= 1ull << x;
      if (p.beta != T(0)) old[x] = d[i * p.d_rs + j * p.d_cs];
    }
  }
#pragma unroll
  for (int x = 0; x < NV; ++x) {
    const T v = p.alpha * acc[x];
    old[x] = p.beta == T(0) ? v : p.beta * old[x] + v;
    asm volatile("" : "+v"(old[x]));  // computed here: not sunk into the store's branch, behind a wait of its own
  }
#pragma unroll
  for (int x = 0; x < NV; ++x) {
    if ((ok >> x) & 1) {
      int64_t i, j;
      at(x, i, j);
      d[i * p.d_rs + j * p.d_cs] = old[x];
    }
  }
}

// ------------------------------------------------------------------------------------------------ VALU path

constexpr int VT = 64, VK = 16;

template <typename T>
__global__ __launch_bounds__(256) void gemm_valu_kernel(GemmProblem<T> p) {
  __shared__ T As[VK][VT + 1];
  __shared__ T Bs[VK][VT + 1];
  const int64_t bi = blockIdx.z;
  const int64_t i0 = (int64_t)blockIdx.y * VT, j0 = (int64_t)blockIdx.x * VT;
  const int64_t i1 = i0 + VT < p.M ? i0 + VT : p.M, j1 = j0 + VT < p.N ? j0 + VT : p.N;
  const TileRange kr = tile_k_range(p, i0, i1, j0, j1);
  if (kr.empty) return;
  const T* a = p.A + bi * p.a_bs;
  const T* b = p.B + bi * p.b_bs;
  T* d = p.D + bi * p.d_bs;
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  T acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = T(0);
  for (int64_t kb = kr.k_lo; kb < kr.k_hi; kb += VK) {
#pragma unroll
    for (int ld = 0; ld < 4; ++ld) {
      const int kl = tid & 15, il = (tid >> 4) + 16 * ld;
      As[kl][il] = load_a(p, a, i0 + il, kb + kl, kr.k_hi);
      const int jl = tid & 63, kl2 = (tid >> 6) + 4 * ld;
      Bs[kl2][jl] = load_b(p, b, kb + kl2, j0 + jl, kr.k_hi);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < VK; ++kk) {
      T av[4], bv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) av[r] = As[kk][ty + 16 * r];
#pragma unroll
      for (int c = 0; c < 4; ++c) bv[c] = Bs[kk][tx + 16 * c];
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[r][c] += av[r] * bv[c];
    }
    __syncthreads();
  }
  T out[16];
#pragma unroll
  for (int x = 0; x < 16; ++x) out[x] = acc[x / 4][x % 4];
  store_d_group(p, d, out, [&](int x, int64_t& i, int64_t& j) {
    i = i0 + ty + 16 * (x / 4);
    j = j0 + tx + 16 * (x % 4);
  });
}

// ------------------------------------------------------------------------------------------------ MFMA path (fp32)

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int MT = 128, MK = 16;

// 256 threads = 4 waves; wave w owns rows 64*(w/2).. and cols 64*(w%2).. of the 128 x 128 tile as
// 2 x 2 blocks of 32 x 32 (v_mfma_f32_32x32x2_f32).  Operand layout of that instruction: lane l
// supplies A(l%32, kslot) and B(kslot, l%32) with kslot = l/32; the 16 accumulators of lane l hold
// D(8*(r/4) + 4*(l/32) + r%4, l%32).  Which k a slot carries is free as long as A and B agree: the
// lane half h takes k = 8*h + s (s = 0..7) over the 8 instructions of one 16-deep K step, so each
// lane reads its 8 values as two 16-byte LDS loads.
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmProblem<float> p) {
  __shared__ __align__(16) float As[MT][MK + 4];  // A(i, k), k fastest
  __shared__ __align__(16) float Bs[MT][MK + 4];  // B(k, j) stored transposed: [j][k]
  const int64_t bi = blockIdx.z;
  const int64_t i0 = (int64_t)blockIdx.y * MT, j0 = (int64_t)blockIdx.x * MT;
  const int64_t i1 = i0 + MT < p.M ? i0 + MT : p.M, j1 = j0 + MT < p.N ? j0 + MT : p.N;
  const TileRange kr = tile_k_range(p, i0, i1, j0, j1);
  if (kr.empty) return;
  const float* a = p.A + bi * p.a_bs;
  const float* b = p.B + bi * p.b_bs;
  float* d = p.D + bi * p.d_bs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int li = lane & 31, half = lane >> 5;
  floatx16 acc[2][2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[r][c][e] = 0.f;

  for (int64_t kb = kr.k_lo; kb < kr.k_hi; kb += MK) {
    // stage 128 x 16 of A and 16 x 128 of B: 2048 values each, 8 per thread
#pragma unroll
    for (int ld = 0; ld < 8; ++ld) {
      const int idx = tid + 256 * ld;
      const int ia = idx / MK, ka = idx % MK;  // A: k fastest across threads when a_cs == 1
      As[ia][ka] = load_a(p, a, i0 + ia, kb + ka, kr.k_hi);
      const int jb = idx % MT, kbb = idx / MT;  // B: j fastest across threads
      Bs[jb][kbb] = load_b(p, b, kb + kbb, j0 + jb, kr.k_hi);
    }
    __syncthreads();
    float4 av[2][2], bv[2][2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float* src = &As[wr + 32 * r + li][8 * half];
      av[r][0] = *reinterpret_cast<const float4*>(src);
      av[r][1] = *reinterpret_cast<const float4*>(src + 4);
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const float* src = &Bs[wc + 32 * c + li][8 * half];
      bv[c][0] = *reinterpret_cast<const float4*>(src);
      bv[c][1] = *reinterpret_cast<const float4*>(src + 4);
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float x = av[r][s >> 2][s & 3], y = bv[c][s >> 2][s & 3];
          acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[r][c], 0, 0, 0);
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {  // two groups of 32 outputs (registers for all 64 at once would spill)
    float out[32];
#pragma unroll
    for (int x = 0; x < 32; ++x) out[x] = acc[r][x / 16][x % 16];
    store_d_group(p, d, out, [&](int x, int64_t& i, int64_t& j) {
      const int c = x / 16, e = x % 16;
      i = i0 + wr + 32 * r + 8 * (e >> 2) + 4 * half + (e & 3);
      j = j0 + wc + 32 * c + li;
    });
  }
}

// ------------------------------------------------------------------------------------------------ MFMA, vectorised

// Fast path for the LDL's problems: A contiguous along k (a_cs == 1), B contiguous along k
// (b_rs == 1, BK) or along j (b_cs == 1), every base pointer 16-byte aligned, every stride and K a
// multiple of 4, so panels move as float4.  Tile 128 x 128, K step 32, register prefetch one step
// ahead, four waves of 64 x 64 (2 x 2 blocks of 32 x 32).  LDS: A as [i][k] (pitch 36), B as
// [j][k] (BK, pitch 36) or [k][j] (pitch 132); the MFMA k-slot of lane half h in MFMA s is
// 16 h + s for both operands.  Structurally zero entries are replaced by 0 element-wise.
constexpr int VKT = 32;

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2.  Re-number them so
// that every XCD receives one contiguous share of the tiles, and walk that share in groups of
// GROUP tile rows, so that concurrently running tiles of one XCD share their A and B panels.
__device__ __forceinline__ void xcd_tile(int64_t gx, int64_t gy, int64_t& tx, int64_t& ty) {
  constexpr int XCDS = 8, GROUP = 8;
  const int64_t n = gx * gy;
  const int64_t lin = (int64_t)blockIdx.y * gx + blockIdx.x;
  const int64_t base = n / XCDS, extra = n % XCDS;
  const int64_t x = lin % XCDS, q = lin / XCDS;
  const int64_t id = x * base + (x < extra ? x : extra) + q;
  const int64_t per_group = GROUP * gx;
  const int64_t g = id / per_group, first = g * GROUP;
  const int64_t rows = gy - first < GROUP ? gy - first : GROUP;
  const int64_t in = id % per_group;
  ty = first + in % rows;
  tx = in / rows;
}

template <bool BK>
__global__ __launch_bounds__(256, 2) void gemm_mfma_vec_kernel(GemmProblem<float> p) {
  constexpr int APITCH = VKT + 4;
  constexpr int BPITCH = BK ? VKT + 4 : MT + 4;
  __shared__ __align__(16) float As[MT * APITCH];
  __shared__ __align__(16) float Bs[BK ? MT * BPITCH : VKT * BPITCH];
  const int64_t bi = blockIdx.z;
  int64_t tx, ty;
  xcd_tile(gridDim.x, gridDim.y, tx, ty);
  const int64_t i0 = ty * MT, j0 = tx * MT;
  const int64_t i1 = i0 + MT < p.M ? i0 + MT : p.M, j1 = j0 + MT < p.N ? j0 + MT : p.N;
  TileRange kr = tile_k_range(p, i0, i1, j0, j1);
  if (kr.empty) return;
  kr.k_lo &= ~int64_t(3);  // float4 granules; the masks zero what lies outside
  const float* a = p.A + bi * p.a_bs;
  const float* b = p.B + bi * p.b_bs;
  float* d = p.D + bi * p.d_bs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = (wave >> 1) * 64, wc = (wave & 1) * 64;
  const int li = lane & 31, hh = lane >> 5;
  floatx16 acc[2][2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[r][c][e] = 0.f;

  float4 ra[4], rb[4];
  auto stage = [&](int64_t kb) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int f = tid + 256 * q;
      {  // A: row ia, k = kb + 4 kq ..
        const int ia = f / (VKT / 4), kq = f % (VKT / 4);
        const int64_t i = i0 + ia, k = kb + 4 * kq;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < p.M && k < kr.k_hi) {
          v = *reinterpret_cast<const float4*>(a + i * p.a_rs + k);
          float* e = reinterpret_cast<float*>(&v);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int64_t kk = k + t;
            const bool z = kk >= kr.k_hi || (p.a_tri == TRI_LOWER && kk > i) || (p.a_tri == TRI_UPPER && kk < i);
            e[t] = z ? 0.f : e[t];
          }
        }
        ra[q] = v;
      }
      if (BK) {  // B(k, j) = b[j * b_cs + k]: row jb of the transposed panel
        const int jb = f / (VKT / 4), kq = f % (VKT / 4);
        const int64_t j = j0 + jb, k = kb + 4 * kq;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < p.N && k < kr.k_hi) {
          v = *reinterpret_cast<const float4*>(b + j * p.b_cs + k);
          float* e = reinterpret_cast<float*>(&v);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int64_t kk = k + t;
            const bool z = kk >= kr.k_hi || (p.b_tri == TRI_LOWER && kk < j) || (p.b_tri == TRI_UPPER && kk > j);
            e[t] = z ? 0.f : e[t];
          }
        }
        rb[q] = v;
      } else {  // B(k, j) = b[k * b_rs + j]: row kk of the panel
        const int kk = f / (MT / 4), jq = f % (MT / 4);
        const int64_t k = kb + kk, j = j0 + 4 * jq;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < kr.k_hi && j < p.N) {
          v = *reinterpret_cast<const float4*>(b + k * p.b_rs + j);
          float* e = reinterpret_cast<float*>(&v);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int64_t jj = j + t;
            const bool z = jj >= p.N || (p.b_tri == TRI_LOWER && k < jj) || (p.b_tri == TRI_UPPER && k > jj);
            e[t] = z ? 0.f : e[t];
          }
        }
        rb[q] = v;
      }
    }
  };

  if (kr.k_lo < kr.k_hi) stage(kr.k_lo);
  for (int64_t kb = kr.k_lo; kb < kr.k_hi; kb += VKT) {
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int f = tid + 256 * q;
      *reinterpret_cast<float4*>(&As[(f / (VKT / 4)) * APITCH + 4 * (f % (VKT / 4))]) = ra[q];
      if (BK)
        *reinterpret_cast<float4*>(&Bs[(f / (VKT / 4)) * BPITCH + 4 * (f % (VKT / 4))]) = rb[q];
      else
        *reinterpret_cast<float4*>(&Bs[(f / (MT / 4)) * BPITCH + 4 * (f % (MT / 4))]) = rb[q];
    }
    __syncthreads();
    if (kb + VKT < kr.k_hi) stage(kb + VKT);
    float4 af[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        af[r][v] = *reinterpret_cast<const float4*>(&As[(wr + 32 * r + li) * APITCH + 16 * hh + 4 * v]);
    if (BK) {
      float4 bf[2][4];
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v)
          bf[c][v] = *reinterpret_cast<const float4*>(&Bs[(wc + 32 * c + li) * BPITCH + 16 * hh + 4 * v]);
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2)
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int c = 0; c < 2; ++c)
            acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[r][s2 >> 2][s2 & 3], bf[c][s2 >> 2][s2 & 3], acc[r][c],
                                                             0, 0, 0);
    } else {
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2) {
        float bv[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) bv[c] = Bs[(16 * hh + s2) * BPITCH + wc + 32 * c + li];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
          for (int c = 0; c < 2; ++c)
            acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[r][s2 >> 2][s2 & 3], bv[c], acc[r][c], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {  // two groups of 32 outputs
    float out[32];
#pragma unroll
    for (int x = 0; x < 32; ++x) out[x] = acc[r][x / 16][x % 16];
    store_d_group(p, d, out, [&](int x, int64_t& i, int64_t& j) {
      const int c = x / 16, e = x % 16;
      i = i0 + wr + 32 * r + 8 * (e >> 2) + 4 * hh + (e & 3);
      j = j0 + wc + 32 * c + li;
    });
  }
}

// ------------------------------------------------------------------------------------------------ MFMA path (fp64)

constexpr int DT = 64, DK = 32;

// Tiles of a problem in the order the kernel takes them, heaviest k range first, so that the shortest tiles
// fill in behind the longest instead of the longest starting last (issued row by row, a triangular operand's
// product took 77% of the dense product's time, not half).  A lower triangular square D takes only its lower
// triangle of tiles (the others would be empty).
enum TileOrder : int32_t {
  ORDER_ROWS = 0,
  ORDER_COLS_UP = 1,
  ORDER_COLS_DOWN = 2,
  ORDER_ROWS_DOWN = 3,
  ORDER_LOWER = 4,
};

__host__ __device__ inline TileOrder tile_order(const GemmProblem<double>& p, int64_t tm, int64_t tn) {
  if (p.a_tri == TRI_NONE && p.b_tri == TRI_NONE && p.d_tri == TRI_LOWER && tm == tn) return ORDER_LOWER;
  if (p.a_tri == TRI_LOWER) return ORDER_ROWS_DOWN;  // work grows with the row
  if (p.a_tri == TRI_NONE && p.b_tri == TRI_LOWER) return ORDER_COLS_UP;  // work falls with the column
  if (p.a_tri == TRI_NONE && p.b_tri == TRI_UPPER) return ORDER_COLS_DOWN;  // work grows with the column
  return ORDER_ROWS;  // equal work, or work falling with the row (A upper)
}

__device__ __forceinline__ void tile_of(TileOrder o, int64_t id, int64_t tm, int64_t tn, int64_t& ti, int64_t& tj) {
  switch (o) {
    case ORDER_LOWER: {  // id = ti (ti + 1) / 2 + tj, tj <= ti
      int64_t r = (int64_t)((__builtin_sqrt(8.0 * (double)id + 1.0) - 1.0) * 0.5);
      while (r * (r + 1) / 2 > id) --r;
      while ((r + 1) * (r + 2) / 2 <= id) ++r;
      ti = r;
      tj = id - r * (r + 1) / 2;
      return;
    }
    case ORDER_COLS_UP: tj = id / tm; ti = id % tm; return;
    case ORDER_COLS_DOWN: tj = tn - 1 - id / tm; ti = id % tm; return;
    case ORDER_ROWS_DOWN: ti = tm - 1 - id / tn; tj = id % tn; return;
    default: ti = id / tn; tj = id % tn; return;
  }
}

// 256 threads = 4 waves; wave w owns the 32 x 32 quadrant (w / 2, w % 2) of the 64 x 64 tile as 2 x 2 blocks
// of v_mfma_f64_16x16x4_f64, whose lane l supplies A(l % 16, l / 16) and B(l / 16, l % 16) and whose
// accumulator element r of lane l holds D(l / 16 + 4 r, l % 16).  K is staged through LDS 32 deep, with the
// next k-block loaded into registers while the current one's MFMAs run; the loads apply the operands'
// triangle masks.
__global__ __launch_bounds__(256) void gemm_mfma64_kernel(GemmProblem<double> p, TileOrder order) {
  typedef double double4_t __attribute__((ext_vector_type(4)));
  constexpr int AL = DT * DK / 256;  // staged entries per thread and operand
  __shared__ double As[DK][DT + 1];
  __shared__ double Bs[DK][DT + 1];
  const int64_t bi = blockIdx.z;
  int64_t ti, tj;
  tile_of(order, blockIdx.x, cdiv(p.M, DT), cdiv(p.N, DT), ti, tj);
  const int64_t i0 = ti * DT, j0 = tj * DT;
  const int64_t i1 = i0 + DT < p.M ? i0 + DT : p.M, j1 = j0 + DT < p.N ? j0 + DT : p.N;
  const TileRange kr = tile_k_range(p, i0, i1, j0, j1);
  if (kr.empty) return;
  const double* a = p.A + bi * p.a_bs;
  const double* b = p.B + bi * p.b_bs;
  double* d = p.D + bi * p.d_bs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, kq = lane >> 4;
  const int wi = 32 * (wave >> 1), wj = 32 * (wave & 1);
  const int ak = tid % DK, ar = tid / DK;  // A entry x: (ar + (256 / DK) x, ak)
  const int bj = tid % DT, bk = tid / DT;  // B entry x: (bk + (256 / DT) x, bj)
  double4_t acc[2][2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[r][c][e] = 0.;
  double ra[AL], rb[AL];
  auto load = [&](int64_t kb) {
#pragma unroll
    for (int x = 0; x < AL; ++x) {
      ra[x] = load_a(p, a, i0 + ar + (256 / DK) * x, kb + ak, kr.k_hi);
      rb[x] = load_b(p, b, kb + bk + (256 / DT) * x, j0 + bj, kr.k_hi);
    }
  };
  if (kr.k_lo < kr.k_hi) load(kr.k_lo);
  for (int64_t kb = kr.k_lo; kb < kr.k_hi; kb += DK) {
#pragma unroll
    for (int x = 0; x < AL; ++x) {
      As[ak][ar + (256 / DK) * x] = ra[x];
      Bs[bk + (256 / DT) * x][bj] = rb[x];
    }
    __syncthreads();
    if (kb + DK < kr.k_hi) load(kb + DK);
    // k slot kq of MFMA s carries k = 16 (kq & 1) + 8 (kq >> 1) + s: the two k-rows that a half-wave's
    // 64-bit reads take together (slots 0 and 1, or 2 and 3) lie 16 rows = 32 banks apart at the odd pitch
    // that keeps the transposing stores above free of conflicts (with k = 4 s + kq they lay 2 banks apart)
    const int kof = 16 * (kq & 1) + 8 * (kq >> 1);
#pragma unroll
    for (int s = 0; s < DK / 4; ++s) {
      double av[2], bv[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) av[r] = As[kof + s][wi + 16 * r + li];
#pragma unroll
      for (int c = 0; c < 2; ++c) bv[c] = Bs[kof + s][wj + 16 * c + li];
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[r][c] = __builtin_amdgcn_mfma_f64_16x16x4f64(av[r], bv[c], acc[r][c], 0, 0, 0);
    }
    __syncthreads();
  }
  double out[16];
#pragma unroll
  for (int x = 0; x < 16; ++x) out[x] = acc[x / 8][(x / 4) % 2][x % 4];
  store_d_group(p, d, out, [&](int x, int64_t& i, int64_t& j) {
    i = i0 + wi + 16 * (x / 8) + kq + 4 * (x % 4);
    j = j0 + wj + 16 * ((x / 4) % 2) + li;
  });
}

// ------------------------------------------------------------------------------------------------ MFMA path (fp64, LDS-direct)

// D = beta D + alpha A B with A's rows and B's rows (BKN: B(k, j) = b[k b_rs + j]) or columns (!BKN: B(k, j) =
// b[j b_cs + k]) contiguous -- the LDL's products.  The tile order, output tile and MFMA blocks of
// gemm_mfma64_kernel; k-tiles of 32 loaded one ahead straight into LDS (128-bit buffer loads with the LDS
// destination bit), double-buffered, one barrier per k-tile.  LDS layouts (as the fp64 outer flush's): a row
// panel (A, and B for !BKN) holds row r's 16 k-pairs at pair positions q ^ (r % 16), so that the 16 rows that
// one cycle of a 128-bit read takes cover the 64 banks; a k-row panel (B for BKN) holds 64 columns per k-row
// plus 16 doubles per 8 k-rows, so that the k-rows k and k + 8 that a half-wave reads together fall 32 banks
// apart.  A k-tile that crosses a triangle's edge or the end of the k range is zeroed where the product may
// not read it, in LDS after it has landed (one more barrier); the others are multiplied as loaded.
constexpr int GT = 64, GK = 32;         // tile edge, k-tile depth (doubles)
constexpr int GBGRP = 512, GBPAD = 16;  // k-row panel: 16 doubles of padding per 8 k-rows of 64

template <bool BKN>
struct Gemm64Lds {
  static constexpr int BSZ = BKN ? GT * GK + GT * GK / GBGRP * GBPAD : GT * GK;
  double a[2][GT * GK];
  double b[2][BSZ];
};

template <bool BKN>
__global__ __launch_bounds__(256, 2) void gemm_mfma64_dma_kernel(GemmProblem<double> p, TileOrder order) {
  typedef double double4_t __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) Gemm64Lds<BKN> sm;
  int64_t ti, tj;
  tile_of(order, blockIdx.x, cdiv(p.M, GT), cdiv(p.N, GT), ti, tj);
  const int64_t i0 = ti * GT, j0 = tj * GT;
  const int64_t i1 = i0 + GT < p.M ? i0 + GT : p.M, j1 = j0 + GT < p.N ? j0 + GT : p.N;
  const TileRange kr = tile_k_range(p, i0, i1, j0, j1);
  if (kr.empty) return;
  const int64_t bi = blockIdx.z;
  const double* a = p.A + bi * p.a_bs;
  const double* b = p.B + bi * p.b_bs;
  double* d = p.D + bi * p.d_bs;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int K = (int)p.K, arows = (int)(i1 - i0), bcols = (int)(j1 - j0);
  const int64_t k_lo = kr.k_lo, k_hi = kr.k_hi;
  const int nt = k_lo < k_hi ? (int)((k_hi - k_lo + GK - 1) / GK) : 0;

  // resources: A from the tile's first row; B (BKN) from each k-tile's first row and the tile's first
  // column, B (!BKN) from the tile's first column
  const __amdgpu_buffer_rsrc_t ra =
      matrix_rsrc(reinterpret_cast<const float*>(a + i0 * p.a_rs), 2 * ((int64_t)(arows - 1) * p.a_rs + K));
  auto b_rsrc = [&](int64_t k0) {
    if constexpr (BKN) {
      const int64_t krows = p.K - k0 < GK ? p.K - k0 : GK;
      return matrix_rsrc(reinterpret_cast<const float*>(b + k0 * p.b_rs + j0), 2 * ((krows - 1) * p.b_rs + bcols));
    } else {
      return matrix_rsrc(reinterpret_cast<const float*>(b + j0 * p.b_cs), 2 * ((int64_t)(bcols - 1) * p.b_cs + K));
    }
  };
  // each wave's four 128-bit loads per panel and k-tile: chunk c = wave + 4 x of 128 doubles (1 KB)
  int aoff[4], boff[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int c = wave + 4 * x;
    const int row = 4 * c + (lane >> 4), kk = 2 * ((lane & 15) ^ (row & 15));  // row panel: row, first k
    aoff[x] = row < arows ? (int)((row * p.a_rs + kk) * 8) : OOB;
    if constexpr (BKN) {
      const int kr2 = 2 * c + (lane >> 5), jj = 2 * (lane & 31);  // k-row panel: k-row, first column
      boff[x] = jj < bcols ? (int)((kr2 * p.b_rs + jj) * 8) : OOB;
    } else {
      boff[x] = row < bcols ? (int)((row * p.b_cs + kk) * 8) : OOB;
    }
  }
  const bool full = arows == GT && bcols == GT;
  // whether k-tile t needs the triangle / k-range pass (uniform)
  auto ragged = [&](int64_t k0) {
    return k0 + GK > k_hi || (p.a_tri == TRI_LOWER && k0 + GK - 1 > i0) || (p.a_tri == TRI_UPPER && k0 < i1 - 1) ||
           (p.b_tri == TRI_LOWER && k0 < j1 - 1) || (p.b_tri == TRI_UPPER && k0 + GK - 1 > j0);
  };
  auto issue = [&](int t, int buf) {
    const int64_t k0 = k_lo + (int64_t)t * GK;
    const __amdgpu_buffer_rsrc_t rb = b_rsrc(k0);
    const int ak = (int)(k0 * 8);
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int f0 = (wave + 4 * x) * 128;
      const int bf0 = BKN ? f0 + f0 / GBGRP * GBPAD : f0;
      if (full && k0 + GK <= p.K) {  // every lane in range: the k offset in the scalar field (which the range
                                     // check does not cover, so never for a k-tile that reaches past K)
        dma_load_so<4>(ra, reinterpret_cast<float*>(&sm.a[buf][f0]), aoff[x], ak);
        if constexpr (BKN)
          dma_load<4>(rb, reinterpret_cast<float*>(&sm.b[buf][bf0]), boff[x]);
        else
          dma_load_so<4>(rb, reinterpret_cast<float*>(&sm.b[buf][bf0]), boff[x], ak);
      } else {
        dma_load<4>(ra, reinterpret_cast<float*>(&sm.a[buf][f0]), aoff[x] == OOB ? OOB : aoff[x] + ak);
        if constexpr (BKN)
          dma_load<4>(rb, reinterpret_cast<float*>(&sm.b[buf][bf0]), boff[x]);
        else
          dma_load<4>(rb, reinterpret_cast<float*>(&sm.b[buf][bf0]), boff[x] == OOB ? OOB : boff[x] + ak);
      }
    }
  };
  // zero what the product may not read in a landed k-tile: k at or past k_hi, and the operands' zero triangles
  auto clear = [&](int t, int buf) {
    const int64_t k0 = k_lo + (int64_t)t * GK;
    for (int f = tid; f < GT * GK; f += 256) {
      const int row = f / GK, q = (f % GK) / 2, e = f % 2;
      const int64_t k = k0 + 2 * (q ^ (row & 15)) + e;  // the element at f of a row panel
      const int64_t i = i0 + row;
      if (k >= k_hi || (p.a_tri == TRI_LOWER && k > i) || (p.a_tri == TRI_UPPER && k < i)) sm.a[buf][f] = 0.;
      if constexpr (BKN) {
        const int kk = f / GT, jj = f % GT;
        const int64_t kb = k0 + kk, j = j0 + jj;
        if (kb >= k_hi || (p.b_tri == TRI_LOWER && kb < j) || (p.b_tri == TRI_UPPER && kb > j))
          sm.b[buf][kk * GT + jj + kk / (GBGRP / GT) * GBPAD] = 0.;
      } else {
        const int64_t j = j0 + row;
        if (k >= k_hi || (p.b_tri == TRI_LOWER && k < j) || (p.b_tri == TRI_UPPER && k > j)) sm.b[buf][f] = 0.;
      }
    }
  };

  double4_t acc[2][2];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[r][c][e] = 0.;
  // fragments: lane (li, hh) supplies A(row 32 wi + 16 a2 + li, k) and B(k, column 32 wj + 16 d2 + li) with
  // k = 8 hh + 2 v + s2 in MFMA (v, s2)
  const int li = lane & 15, hh = lane >> 4;
  const int wi = wave >> 1, wj = wave & 1;
  const int a_base = (32 * wi + li) * GK;
  const int b_base = BKN ? 8 * hh * GT + 32 * wj + li + hh * GBPAD : (32 * wj + li) * GK;
  auto step = [&](int t, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    __syncthreads();  // buffer cur has landed; buffer 1 - cur is no longer read
    if (ragged(k_lo + (int64_t)t * GK)) {
      clear(t, cur);
      __syncthreads();
    }
    if (t + 1 < nt) issue(t + 1, 1 - cur);
    const double* as = &sm.a[cur][a_base];
    const double* bs = &sm.b[cur][b_base];
    double2 fa[2][2], fbv[2][2];  // [slot][block]
    double fb[2][2][2];           // [slot][block][s2] (BKN)
    auto frag = [&](int v, int slot) {
#pragma unroll
      for (int a2 = 0; a2 < 2; ++a2)
        fa[slot][a2] = *reinterpret_cast<const double2*>(as + a2 * 16 * GK + 2 * ((4 * hh + v) ^ li));
#pragma unroll
      for (int d2 = 0; d2 < 2; ++d2) {
        if constexpr (BKN) {
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) fb[slot][d2][s2] = bs[16 * d2 + (2 * v + s2) * GT];
        } else {
          fbv[slot][d2] = *reinterpret_cast<const double2*>(bs + d2 * 16 * GK + 2 * ((4 * hh + v) ^ li));
        }
      }
    };
    frag(0, 0);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      if (v < 3) frag(v + 1, (v + 1) & 1);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2)
#pragma unroll
          for (int d2 = 0; d2 < 2; ++d2) {
            const double av = s2 ? fa[v & 1][a2].y : fa[v & 1][a2].x;
            double bv;
            if constexpr (BKN)
              bv = fb[v & 1][d2][s2];
            else
              bv = s2 ? fbv[v & 1][d2].y : fbv[v & 1][d2].x;
            acc[a2][d2] = __builtin_amdgcn_mfma_f64_16x16x4f64(av, bv, acc[a2][d2], 0, 0, 0);
          }
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_dma();  // this wave's loads of k-tile t + 1 have landed before the next barrier
  };
  if (nt > 0) {
    issue(0, 0);
    wait_dma();
    for (int t = 0; t < nt; t += 2) {
      step(t, std::integral_constant<int, 0>{});
      if (t + 1 < nt) step(t + 1, std::integral_constant<int, 1>{});
    }
  }
  double out[16];
#pragma unroll
  for (int x = 0; x < 16; ++x) out[x] = acc[x / 8][(x / 4) % 2][x % 4];
  store_d_group(p, d, out, [&](int x, int64_t& i, int64_t& j) {
    i = i0 + 32 * wi + 16 * (x / 8) + hh + 4 * (x % 4);
    j = j0 + 32 * wj + 16 * ((x / 4) % 2) + li;
  });
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// The LDS-direct fp64 path applies: A's rows and B's rows (bkn) or columns contiguous, every row stride, batch
// stride and K in whole 16-byte pairs, both operands on 16-byte boundaries, and every byte offset inside a
// 64-row (or 32 k-row) panel below 2^30.
bool dma64_ok(const GemmProblem<double>& p, bool& bkn) {
  constexpr int64_t lim = (int64_t)1 << 27;  // doubles
  if (p.a_cs != 1 || p.a_rs <= 0 || p.a_rs % 2 || p.a_bs % 2 || !aligned16(p.A)) return false;
  if (p.K <= 0 || p.K % 2 || GT * p.a_rs + p.K >= lim || !aligned16(p.B) || p.b_bs % 2) return false;
  if (p.b_cs == 1 && p.b_rs > 0 && p.b_rs % 2 == 0 && p.N % 2 == 0 && GK * p.b_rs + p.N < lim) {
    bkn = true;
    return true;
  }
  if (p.b_rs == 1 && p.b_cs > 0 && p.b_cs % 2 == 0 && GT * p.b_cs + p.K < lim) {
    bkn = false;
    return true;
  }
  return false;
}

// The vectorised path applies: strides, offsets and the K extent in float4 granules.
bool vec_ok(const GemmProblem<float>& p, bool& bk) {
  if (p.a_cs != 1 || p.a_rs % 4 || p.a_bs % 4 || !aligned16(p.A)) return false;
  if (!aligned16(p.B) || p.b_bs % 4 || p.K % 4) return false;
  if (p.b_rs == 1 && p.b_cs % 4 == 0) bk = true;
  else if (p.b_cs == 1 && p.b_rs % 4 == 0 && p.N % 4 == 0) bk = false;
  else return false;
  return p.M >= MT / 2 && p.N >= MT / 2;
}

}  // namespace

template <typename T>
int gptq2d_gemm(const GemmProblem<T>& p, hipStream_t stream) {
  if (p.M < 0 || p.N < 0 || p.K < 0 || p.batch < 0) return GPTQ2D_EINVAL;
  if (p.M == 0 || p.N == 0 || p.batch == 0) return 0;
  if (p.batch > 65535) return GPTQ2D_EUNSUPPORTED;
  if constexpr (sizeof(T) == 8) {
    const int64_t tm = cdiv(p.M, DT), tn = cdiv(p.N, DT);
    const TileOrder order = tile_order(p, tm, tn);
    const int64_t tiles = order == ORDER_LOWER ? tm * (tm + 1) / 2 : tm * tn;
    if (tiles > 0x7fffffff) return GPTQ2D_EUNSUPPORTED;
    const dim3 grid((unsigned)tiles, 1u, (unsigned)p.batch);
    bool bkn = false;
    if (dma64_ok(p, bkn)) {
      if (bkn)
        hipLaunchKernelGGL(gemm_mfma64_dma_kernel<true>, grid, dim3(256), 0, stream, p, order);
      else
        hipLaunchKernelGGL(gemm_mfma64_dma_kernel<false>, grid, dim3(256), 0, stream, p, order);
    } else {
      hipLaunchKernelGGL(gemm_mfma64_kernel, grid, dim3(256), 0, stream, p, order);
    }
    return (int)hipGetLastError();
  } else {
    bool bk = false;
    if (vec_ok(p, bk)) {
      const dim3 grid((unsigned)cdiv(p.N, MT), (unsigned)cdiv(p.M, MT), (unsigned)p.batch);
      if (bk)
        hipLaunchKernelGGL(gemm_mfma_vec_kernel<true>, grid, dim3(256), 0, stream, p);
      else
        hipLaunchKernelGGL(gemm_mfma_vec_kernel<false>, grid, dim3(256), 0, stream, p);
      return (int)hipGetLastError();
    }
    if (p.M >= MT / 2 && p.N >= MT / 2) {
      const dim3 grid((unsigned)cdiv(p.N, MT), (unsigned)cdiv(p.M, MT), (unsigned)p.batch);
      hipLaunchKernelGGL(gemm_mfma_kernel, grid, dim3(256), 0, stream, p);
      return (int)hipGetLastError();
    }
  }
  const dim3 grid((unsigned)cdiv(p.N, VT), (unsigned)cdiv(p.M, VT), (unsigned)p.batch);
  hipLaunchKernelGGL(gemm_valu_kernel<T>, grid, dim3(256), 0, stream, p);
  return (int)hipGetLastError();
}

template int gptq2d_gemm<float>(const GemmProblem<float>&, hipStream_t);
template int gptq2d_gemm<double>(const GemmProblem<double>&, hipStream_t);

extern "C" {

// The strided GEMM as a C entry point, so that tests can check both paths (and the MFMA operand
// layout) against a host product.  No counterpart in the reference.
#define GPTQ2D_GEMM_ABI(SUF, T)                                                                                     \
  int gptq2d_gemm_##SUF(int64_t M, int64_t N, int64_t K, int64_t batch, const T* A, int64_t a_rs, int64_t a_cs,    \
                        int64_t a_bs, const T* B, int64_t b_rs, int64_t b_cs, int64_t b_bs, T* D, int64_t d_rs,     \
                        int64_t d_cs, int64_t d_bs, double alpha, double beta, int32_t a_tri, int32_t b_tri,       \
                        int32_t d_tri, hipStream_t stream) {                                                       \
    if (a_tri < 0 || a_tri > 2 || b_tri < 0 || b_tri > 2 || d_tri < 0 || d_tri > 2) return GPTQ2D_EINVAL;          \
    GemmProblem<T> p{M, N, K, batch, A, a_rs, a_cs, a_bs, B, b_rs, b_cs, b_bs, D, d_rs, d_cs, d_bs,               \
                     (T)alpha, (T)beta, a_tri, b_tri, d_tri};                                                      \
    return gptq2d_gemm<T>(p, stream);                                                                                \
  }

GPTQ2D_GEMM_ABI(f32, float)
GPTQ2D_GEMM_ABI(f64, double)

}  // extern "C"
