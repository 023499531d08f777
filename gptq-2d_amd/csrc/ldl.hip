// Feedback-factor preprocessing: the (block) LDL factor of a Kronecker factor's inverse.
//
// ldl_of_inverse(M, size) returns the unit lower (block) triangular L with M^{-1} = L Lambda L^T
// (Lambda block diagonal with size x size blocks) without forming M^{-1}: with J the reversal,
// the Cholesky factor C of J M J (lower, J M J = C C^T) gives Um = J C J, upper, M = Um Um^T, and
// L_raw = Um^{-T} = J C^{-T} J, i.e. L_raw(i, j) = C^{-1}(k-1-j, k-1-i).  L is L_raw normalised by
// its diagonal (size 1) or, for size p, (L_raw - D) D^{-1} + I with D the p x p block diagonal.
// ldl(M, size) is the same normalisation applied to the Cholesky factor of M itself.
//
// Device work, all on the caller's stream, no host synchronisation, no device allocation by this
// library:
//   1. W = J M J: the reversal of the flat array.
//   2. Right-looking blocked Cholesky of W in place, panels of PB columns: a panel's diagonal
//      block is factored (redundantly in every workgroup) and the panel below solved against it;
//      the trailing lower triangle takes the rank-PB update.  fp32 (k % 4 == 0) blocks it on two
//      levels: strips of 8 panels (16 from k = 8192), where each panel updates only its strip's later
//      columns and a strip's end brings one update of the whole trailing triangle of the strip's rank
//      (512 or 1024; MFMA-bound, where
//      rank-64 updates are bound by moving the triangle through HBM), with a look-ahead of one
//      panel on the one stream: after a panel, a strip launch updates only the next panel's
//      columns, and the next panel's factorisation shares one launch (panel_step_kernel) with the
//      rest of the update, on disjoint columns -- the latency-bound panel runs beside the MFMA
//      update instead of after it.  fp64 (and fp32 with k % 4 != 0) keep the plain sequence, the
//      update on gemm.hip.
//   3. ldl_of_inverse only: C^{-1} in place by recursive doubling.  Diagonal NB blocks are inverted
//      by one wave each; then for s = NB, 2 NB, ... every pair of inverted s-blocks A^{-1}, D^{-1}
//      with off-diagonal block B becomes one inverted 2s-block through -D^{-1} (B A^{-1}) -- two
//      triangular GEMMs per level, all pairs of a level in one batched launch.  For fp32 with
//      16-byte aligned rows they run on the triangular MFMA GEMM of trmm_mfma.hip (each block's
//      k loop restricted to the k-tiles that meet the triangular operand's non-zero part), otherwise
//      on the strided GEMM of gemm.hip; the unused part of the output buffer holds the products.
//      No vendor library is called.
//   4. Normalisation into L (LDS-tiled transposed read for ldl_of_inverse).
//
// A non-positive (or NaN) pivot records its 1-based column in `info` (device int, 0 when the
// factorisation succeeded); the numbers that follow are then meaningless, as in LAPACK.
//
// Reference: IST-DASLab/GPTQ-2D gptq_2d_reference.py:29-55 (_unit_diagonal_blocks, ldl_of_inverse,
// ldl), which call torch.linalg.cholesky and solve_triangular.
#include "linalg.h"
#include "lds_dma.h"


#include <array>
#include <type_traits>
#include <unordered_map>
#include <utility>

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

template <typename T>
struct LdlBlock;
// NB: diagonal blocks inverted by one wave in registers (trtri leaves, block normalisation);
// PB: Cholesky panel width (the diagonal block is factored in LDS).
template <>
struct LdlBlock<float> {
  static constexpr int NB = 64;
  static constexpr int PB = 64;
  static constexpr int SB = 128;  // largest diagonal block of the block normalisation (LDS solve above NB)
};
template <>
struct LdlBlock<double> {
  static constexpr int NB = 32;
  static constexpr int PB = 32;
  static constexpr int SB = 64;
};

__device__ __forceinline__ float bcast(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ double bcast(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Lane r holds row r of an NB x NB lower triangular block in a; returns row r of its inverse in x.
template <typename T, int NB>
__device__ __forceinline__ void wave_trtri(const T (&a)[NB], T (&x)[NB], int lane) {
  T dg = T(1);
#pragma unroll
  for (int c = 0; c < NB; ++c)
    if (c == lane) dg = a[c];
  T acc[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c) acc[c] = T(0);
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    // row t of the inverse: (e_t - acc_t) / C(t, t), acc_t complete since every row u < t is in
    const T inv_t = T(1) / bcast(dg, t);
#pragma unroll
    for (int c = 0; c <= t; ++c) {
      const T xt = ((c == t ? T(1) : T(0)) - bcast(acc[c], t)) * inv_t;
      if (lane > t) acc[c] += a[t] * xt;
    }
  }
  const T inv = T(1) / dg;
#pragma unroll
  for (int c = 0; c < NB; ++c) x[c] = c <= lane ? ((c == lane ? T(1) : T(0)) - acc[c]) * inv : T(0);
}

// dst = src (rev = 0) or dst = the reversal of the flat src (rev = 1), which is J M J for a matrix;
// info[0..n_info) = 0 (the pivot report of the factorisation that follows on the same stream).
template <typename T>
__global__ void copy_kernel(T* __restrict__ dst, const T* __restrict__ src, int64_t count, int rev,
                            int* __restrict__ info, int n_info) {
  if (blockIdx.x == 0 && (int)threadIdx.x < n_info) info[threadIdx.x] = 0;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < count; t += (int64_t)gridDim.x * blockDim.x)
    dst[t] = src[rev ? count - 1 - t : t];
}

// info[0..n) = 0 where no copy precedes the factorisation (empty matrices).
__global__ void zero_info_kernel(int* __restrict__ info, int64_t n) {
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += (int64_t)gridDim.x * blockDim.x)
    info[t] = 0;
}

// Value of lane (lane & ~3) | O for every lane of each quad (DPP quad_perm, no LDS).
template <int O>
__device__ __forceinline__ float quad_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), O | (O << 2) | (O << 4) | (O << 6), 0xf, 0xf,
                                                 false));
}
template <int O>
__device__ __forceinline__ double quad_bcast(double v) {
  const long long b = __double_as_longlong(v);
  constexpr int ctl = O | (O << 2) | (O << 4) | (O << 6);
  const int lo = __builtin_amdgcn_mov_dpp((int)(b & 0xffffffffll), ctl, 0xf, 0xf, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), ctl, 0xf, 0xf, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

template <int T0, int PB, typename T>
__device__ __forceinline__ void quad_solve_step(T (&x)[PB / 4], int q, const T* __restrict__ a, int cp,
                                                const T* __restrict__ rinv) {
  // column T0: its owner (lane q == T0 % 4, slot T0 / 4) finalises x_T0 (times the pivot's
  // reciprocal), the quad shares it, and every lane removes it from its own later columns
  // c = 4 idx + q > T0
  constexpr int O = T0 & 3, IT = T0 >> 2;
  T xt = x[IT] * rinv[T0];
  xt = quad_bcast<O>(xt);
  if (q == O) x[IT] = xt;
#pragma unroll
  for (int idx = IT; idx < PB / 4; ++idx) {
    const int c = 4 * idx + q;
    if (c > T0) x[idx] -= xt * a[c * cp + T0];
  }
}

template <int T0, int PB, typename T>
__device__ __forceinline__ void quad_solve(T (&x)[PB / 4], int q, const T* __restrict__ a, int cp,
                                           const T* __restrict__ rinv) {
  if constexpr (T0 < PB) {
    quad_solve_step<T0, PB, T>(x, q, a, cp, rinv);
    quad_solve<T0 + 1, PB, T>(x, q, a, cp, rinv);
  }
}

// fp32 step T0 (0 .. 15) of a 16-column block of the solve below, with the block's coefficients in
// registers: cf[j][t] = C(c, c0 + t) for the lane's column c = c0 + 4 j + q when c > c0 + t, else 0
// (so the finished entries and the owner's own entry take x - xt * 0 = x), ri[t] = 1 / C(t, t).
template <int T0>
__device__ __forceinline__ void block16_step(float (&x)[4], const float (&cf)[4][16], const float (&ri)[16], int q) {
  constexpr int O = T0 & 3, IT = T0 >> 2;
  float xt = x[IT] * ri[T0];
  xt = quad_bcast<O>(xt);
  if (q == O) x[IT] = xt;
#pragma unroll
  for (int j = IT; j < 4; ++j) x[j] -= xt * cf[j][T0];
}
template <int... Ts>
__device__ __forceinline__ void block16_steps(float (&x)[4], const float (&cf)[4][16], const float (&ri)[16], int q,
                                              std::integer_sequence<int, Ts...>) {
  (block16_step<Ts>(x, cf, ri, q), ...);
}

// Pivot of a Cholesky column: sd = sqrt(d) and inv = 1 / sd.  fp32: the hardware reciprocal square
// root refined by one Newton step, y (3 - d y^2) / 2, so that the column is scaled by a product, not a
// quotient (the dependent chain of every column is the panel's critical path).
__device__ __forceinline__ void pivot(float d, float& sd, float& inv) {
  const float y = __builtin_amdgcn_rsqf(d);
  inv = y * fmaf(-0.5f * d * y, y, 1.5f);
  sd = d * inv;
}
__device__ __forceinline__ void pivot(double d, double& sd, double& inv) {
  sd = sqrt(d);
  inv = 1.0 / sd;
}

// One panel of the blocked Cholesky.  Every workgroup factors the diagonal block W[j0.., j0..]
// (n = min(PB, k - j0) rows; rows beyond n act as identity rows): the block is staged through LDS
// with coalesced loads and factored 16 columns at a time -- one wave factors the 16 columns in
// registers, lane r holding row r, column by column with no barrier (the pivot and the scaled
// column entries reach the other lanes by readlane; lane r's entries right of its diagonal take
// harmless updates and are never read), then the workgroup applies the rank-16 update to the
// block's later columns (fp32: one 32 x 32 MFMA tile per wave); the workgroups stage the factored
// block.  Then the panel below is solved against it, W[r, j0:j0+PB] <- W[r, j0:j0+PB] C_jj^{-T}, in
// chunks of 64 rows staged through LDS (coalesced loads and stores; a workgroup's first chunk is
// loaded into registers before the factorisation, so the load overlaps it): four lanes share a
// row, lane q owning the columns c = q mod 4, and the forward substitution runs column by column
// with the finished x_t broadcast inside the quad (fp32: in blocks of 16 columns with the block's
// coefficients in registers and the updates between blocks on MFMA, solve_chunk16).
template <typename T, int PB>
struct PotrfLds {
  static constexpr int CP = PB + 1;  // odd pitch: row and column walks are both conflict-free
  T a[PB * CP];
  T rs[64 * CP];
  T rinv[PB];  // reciprocals of the factored block's diagonal
  T pd[PB * CP];  // the update's source panel: the rows of the diagonal block
  T px[64 * CP];  // and the rows of the current chunk
};

// Lane layout of a 64 x 64 product on MFMA (v_mfma_f32_32x32x2_f32) from row-major LDS operands
// with pitch cp: wave (wy, wx) forms the 32 x 32 tile at rows 32 wy, columns 32 wx of A B^T (K = 64,
// k = 2 s + h for MFMA s), acc[e] = tile(8 (e / 4) + 4 h + e % 4, lane % 32).
__device__ __forceinline__ floatx16 tile_abt64(const float* __restrict__ A, const float* __restrict__ B, int cp,
                                               int wy, int wx, int li, int hh) {
  // every operand read before the first MFMA: no LDS latency between MFMAs
  float av[32], bv[32];
#pragma unroll
  for (int s2 = 0; s2 < 32; ++s2) {
    av[s2] = A[(32 * wy + li) * cp + 2 * s2 + hh];
    bv[s2] = B[(32 * wx + li) * cp + 2 * s2 + hh];
  }
  floatx16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
  for (int s2 = 0; s2 < 32; ++s2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s2], bv[s2], acc, 0, 0, 0);
  return acc;
}

// fp32 solve of a 64-row chunk, X <- X C^{-T} (X: 64 x 64 in rs, C: the factored 64 x 64 block in a,
// rinv: its diagonal's reciprocals), in four blocks of 16 columns.  Inside a block, the forward
// substitution of quad_solve (four lanes per row, lane q owning the columns c = q mod 4) with the
// block's coefficients read into registers first, so that no LDS read sits in its 16-step chain;
// then the block's rank-16 update of the later columns, X[:, later] -= X[:, block] C[later, block]^T,
// on MFMA (wave (wy, wx): the 32 x 32 tile at rows 32 wy, columns 32 wx, when it holds later
// columns).  Expects rs complete (a barrier after it was written); ends with a barrier.
__device__ __forceinline__ void solve_chunk16(float* __restrict__ rs, const float* __restrict__ a,
                                              const float* __restrict__ rinv, int tid) {
  constexpr int CP = 65;
  const int q = tid & 3, rr = tid >> 2;
  const int lane = tid & 63, li = lane & 31, hh = lane >> 5, wy = tid >> 7, wx = (tid >> 6) & 1;
  // block b's coefficients, read one block ahead (they do not depend on the chunk)
  float cf[2][4][16], ri[2][16];
  auto coefs = [&](int b, int slot) {
    const int c0 = 16 * b;
#pragma unroll
    for (int t = 0; t < 16; ++t) ri[slot][t] = rinv[c0 + t];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < 4 * j + 4; ++t)
        cf[slot][j][t] = 4 * j + q > t ? a[(c0 + 4 * j + q) * CP + c0 + t] : 0.f;
  };
  coefs(0, 0);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int c0 = 16 * b;
    float x[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = rs[rr * CP + c0 + 4 * j + q];
    if (b < 3) coefs(b + 1, (b + 1) & 1);
    block16_steps(x, cf[b & 1], ri[b & 1], q, std::make_integer_sequence<int, 16>{});
#pragma unroll
    for (int j = 0; j < 4; ++j) rs[rr * CP + c0 + 4 * j + q] = x[j];
    __syncthreads();
    if (b < 3) {
      if (32 * wx + 31 >= c0 + 16) {
        float av[8], bv[8];
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) {
          av[s2] = rs[(32 * wy + li) * CP + c0 + 2 * s2 + hh];
          bv[s2] = a[(32 * wx + li) * CP + c0 + 2 * s2 + hh];
        }
        floatx16 acc;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < 8; ++s2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s2], bv[s2], acc, 0, 0, 0);
        const int col = 32 * wx + li;
        if (col >= c0 + 16) {
#pragma unroll
          for (int e = 0; e < 16; ++e) rs[(32 * wy + 8 * (e >> 2) + 4 * hh + (e & 3)) * CP + col] -= acc[e];
        }
      }
      __syncthreads();
    }
  }
}

// Panel j0 as above, for workgroup `bid` of `nblk` taking part (the panel's row chunks are dealt
// over them).
template <typename T, int PB>
__device__ __forceinline__ void potrf_panel(PotrfLds<T, PB>& sm, T* __restrict__ w, int64_t ld, int64_t j0, int n,
                                            int64_t k, int* __restrict__ info, T* __restrict__ stage, int64_t bid,
                                            int64_t nblk, int64_t upc = -1) {
  // upc >= 0 (fp32): the panel's columns still lack the rank-PB update of the panel at columns
  // [upc, upc + PB); the workgroup applies it to the diagonal block and to each of its chunks (on
  // MFMA, before the factorisation and before each solve) instead of a launch of its own
  constexpr int CP = PB + 1;
  constexpr bool kFuse = sizeof(T) == 4 && PB == 64;
  const bool fuse = kFuse && upc >= 0;
  T* a = sm.a;
  T* rs = sm.rs;
  const int tid = threadIdx.x;
  const int lane = tid & 63, li = lane & 31, hh = lane >> 5, wy = tid >> 7, wx = (tid >> 6) & 1;
  // every load of the prologue is issued before any is waited for (into registers, unrolled): a
  // load-then-store loop would wait out one memory latency per element.
  // Lane (rl, cl) = (tid / PB, tid % PB) loads rows rl + RS u of column cl.  A full panel (n = PB)
  // loads unconditionally along one pointer (the upper triangle's values are read and dropped);
  // the last, short panel takes the guarded walk.
  constexpr int NL = PB * PB / 256, RS = 256 / PB;
  const int rl = tid / PB, cl = tid % PB;
  T dv[NL], pv[NL];
  if (n == PB) {
    const T* src = w + (j0 + rl) * ld + j0 + cl;
    const T* psrc = w + (j0 + rl) * ld + upc + cl;
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const T v = src[(int64_t)u * RS * ld];
      dv[u] = cl <= rl + RS * u ? v : T(0);
      if (fuse) pv[u] = psrc[(int64_t)u * RS * ld];
    }
  } else {
#pragma unroll
    for (int u = 0; u < NL; ++u) {
      const int t = tid + 256 * u, r = t / PB, c = t % PB;
      dv[u] = (r < n && c <= r) ? w[(j0 + r) * ld + j0 + c] : (r == c ? T(1) : T(0));
      if (fuse) pv[u] = r < n ? w[(j0 + r) * ld + upc + c] : T(0);
    }
  }
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int t = tid + 256 * u, r = t / PB, c = t % PB;
    a[r * CP + c] = dv[u];
    if (fuse) sm.pd[r * CP + c] = pv[u];
  }
  __syncthreads();
  // this workgroup's first chunk of the panel below (and of the update's source panel), in flight
  // during the factorisation.  Issued only now: every workgroup of the launch reads the same
  // diagonal block (cache hits after the first) but a chunk of its own, and chunk loads issued
  // beside the block's would hold the factorisation's start behind the whole launch's chunk traffic
  const int64_t first = j0 + PB;
  constexpr int PRE = 64 * PB / 256;
  T pre[PRE], xpre[PRE];
  if (n == PB) {
    const int64_t r0 = first + bid * 64;
    if (r0 + 64 <= k) {
      const T* src = w + (r0 + rl) * ld + j0 + cl;
      const T* psrc = w + (r0 + rl) * ld + upc + cl;
#pragma unroll
      for (int u = 0; u < PRE; ++u) {
        pre[u] = src[(int64_t)u * RS * ld];
        if (fuse) xpre[u] = psrc[(int64_t)u * RS * ld];
      }
    } else {
#pragma unroll
      for (int u = 0; u < PRE; ++u) {
        const int t = tid + 256 * u, i = t / PB, c = t % PB;
        pre[u] = r0 + i < k ? w[(r0 + i) * ld + j0 + c] : T(0);
        if (fuse) xpre[u] = r0 + i < k ? w[(r0 + i) * ld + upc + c] : T(0);
      }
    }
  }
  if constexpr (kFuse) {
    if (fuse) {
      // the diagonal block: a -= Pd Pd^T (the tile above the diagonal is not needed)
      if (wy >= wx) {
        const floatx16 acc = tile_abt64(sm.pd, sm.pd, CP, wy, wx, li, hh);
#pragma unroll
        for (int e = 0; e < 16; ++e) a[(32 * wy + 8 * (e >> 2) + 4 * hh + (e & 3)) * CP + 32 * wx + li] -= acc[e];
      }
      __syncthreads();
    }
  }
  constexpr int CB = 16;
  int bad = 0;
#pragma unroll
  for (int c0 = 0; c0 < PB; c0 += CB) {
    if (tid < 64) {
      const int r = tid < PB ? tid : PB - 1;
      T x[CB], myinv = T(0);
#pragma unroll
      for (int c = 0; c < CB; ++c) x[c] = a[r * CP + c0 + c];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        const T d = bcast(x[c], c0 + c);
        if (!(d > T(0)) && bad == 0) bad = c0 + c + 1;
        T sd, inv;
        pivot(d, sd, inv);
        if (tid == c0 + c) myinv = inv;
        // fp32: the pivot lane's x[c] is d, and d * inv is sd bit for bit (pivot), so no select
        x[c] = (sizeof(T) == 4 || tid != c0 + c) ? x[c] * inv : sd;
#pragma unroll
        for (int c2 = c + 1; c2 < CB; ++c2) x[c2] -= x[c] * bcast(x[c], c0 + c2);
      }
      if (tid < PB && tid >= c0) {
#pragma unroll
        for (int c = 0; c < CB; ++c) a[r * CP + c0 + c] = x[c];
        if (tid < c0 + CB) sm.rinv[tid] = myinv;
      }
    }
    __syncthreads();
    if (c0 + CB < PB) {
      // a[r][c2] -= sum_{c in block} a[r][c] a[c2][c] for the later columns c2 >= c0 + CB (every row:
      // the entries above the diagonal take harmless updates)
      if constexpr (sizeof(T) == 4 && PB == 64) {
        // wave (wy, wx): the 32 x 32 tile at rows 32 wy, columns 32 wx; 8 MFMAs of k-depth 2, lane
        // (i, h) feeding k = c0 + 2 s + h of row 32 wy + i (A) and of row 32 wx + i (B)
        const int lane = tid & 63, li = lane & 31, hh = lane >> 5;
        const int wy = tid >> 7, wx = (tid >> 6) & 1;
        if (32 * wx + 31 >= c0 + CB) {
          float av[CB / 2], bv[CB / 2];
#pragma unroll
          for (int s2 = 0; s2 < CB / 2; ++s2) {
            av[s2] = a[(32 * wy + li) * CP + c0 + 2 * s2 + hh];
            bv[s2] = a[(32 * wx + li) * CP + c0 + 2 * s2 + hh];
          }
          floatx16 acc;
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[e] = 0.f;
#pragma unroll
          for (int s2 = 0; s2 < CB / 2; ++s2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s2], bv[s2], acc, 0, 0, 0);
          const int col = 32 * wx + li;
          if (col >= c0 + CB) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const int row = 32 * wy + 8 * (e >> 2) + 4 * hh + (e & 3);
              a[row * CP + col] -= acc[e];
            }
          }
        }
      } else {
        for (int e = tid; e < PB * PB; e += 256) {
          const int r = e / PB, c2 = e % PB;
          if (c2 < c0 + CB || c2 > r) continue;
          T acc = a[r * CP + c2];
#pragma unroll
          for (int c = 0; c < CB; ++c) acc -= a[r * CP + c0 + c] * a[c2 * CP + c0 + c];
          a[r * CP + c2] = acc;
        }
      }
      __syncthreads();
    }
  }
  if (bid == 0 && tid == 0 && bad && info[0] == 0) info[0] = (int)(j0 + bad);
  // the factored block goes to the staging block, not back into W: workgroups of this launch that
  // start late (the GPU busy with other work) still read the unfactored block from W; a later
  // launch copies it into W (stage_to_w)
  // (its rows dealt over the launch's workgroups: row r by workgroup r mod nblk)
  for (int r = (int)(bid % PB); r < n; r += (int)(nblk < PB ? nblk : PB))
    if (bid < PB && tid <= r) stage[r * n + tid] = a[r * CP + tid];  // pitch n: fits any k x k buffer
  if (n < PB) return;
  const int q = tid & 3, rr = tid >> 2;
  for (int64_t r0 = first + bid * 64; r0 < k; r0 += nblk * 64) {
    __syncthreads();
    if (r0 == first + bid * 64) {
#pragma unroll
      for (int u = 0; u < PRE; ++u) {
        const int t = tid + 256 * u, i = t / PB, c = t % PB;
        rs[i * CP + c] = pre[u];
        if (fuse) sm.px[i * CP + c] = xpre[u];
      }
    } else {
      for (int t = tid; t < 64 * PB; t += 256) {
        const int i = t / PB, c = t % PB;
        rs[i * CP + c] = r0 + i < k ? w[(r0 + i) * ld + j0 + c] : T(0);
        if (fuse) sm.px[i * CP + c] = r0 + i < k ? w[(r0 + i) * ld + upc + c] : T(0);
      }
    }
    __syncthreads();
    if constexpr (kFuse) {
      if (fuse) {
        // the chunk: X -= Px Pd^T
        const floatx16 acc = tile_abt64(sm.px, sm.pd, CP, wy, wx, li, hh);
#pragma unroll
        for (int e = 0; e < 16; ++e) rs[(32 * wy + 8 * (e >> 2) + 4 * hh + (e & 3)) * CP + 32 * wx + li] -= acc[e];
        __syncthreads();
      }
    }
    if constexpr (kFuse) {
      solve_chunk16(rs, a, sm.rinv, tid);
    } else {
      T x[PB / 4];
#pragma unroll
      for (int idx = 0; idx < PB / 4; ++idx) x[idx] = rs[rr * CP + 4 * idx + q];
      quad_solve<0, PB, T>(x, q, a, CP, sm.rinv);
#pragma unroll
      for (int idx = 0; idx < PB / 4; ++idx) rs[rr * CP + 4 * idx + q] = x[idx];
      __syncthreads();
    }
    for (int t = tid; t < 64 * PB; t += 256) {
      const int i = t / PB, c = t % PB;
      if (r0 + i < k) w[(r0 + i) * ld + j0 + c] = rs[i * CP + c];
    }
  }
}

// The staged factored diagonal block of panel j0 (n rows) into W, by one workgroup.
template <typename T, int PB>
__device__ __forceinline__ void stage_to_w(T* __restrict__ w, int64_t ld, int64_t j0, int n,
                                           const T* __restrict__ stage) {
  // all loads issued before the first store (256 threads; a load-then-store loop would wait out one
  // memory latency per element)
  constexpr int NL = PB * PB / 256;
  T v[NL];
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int t = threadIdx.x + 256 * u, r = t / PB, c = t % PB;
    v[u] = (r < n && c <= r) ? stage[r * n + c] : T(0);
  }
#pragma unroll
  for (int u = 0; u < NL; ++u) {
    const int t = threadIdx.x + 256 * u, r = t / PB, c = t % PB;
    if (r < n && c <= r) w[(j0 + r) * ld + j0 + c] = v[u];
  }
}

// Panel j0 of the one-panel-per-launch Cholesky.  copy != nullptr: the last workgroup moves the staged block of
// an earlier panel (at column copy_j0, copy_n rows; another staging slot) into W instead -- the block no
// launch between the two panels reads, so that it needs no launch of its own.
template <typename T, int PB>
__global__ __launch_bounds__(256) void potrf_panel_kernel(T* __restrict__ w, int64_t ld, int64_t j0, int n,
                                                          int64_t k, int* __restrict__ info, T* __restrict__ stage,
                                                          const T* __restrict__ copy, int64_t copy_j0, int copy_n) {
  __shared__ PotrfLds<T, PB> sm;
  const bool copier = copy != nullptr && blockIdx.x == gridDim.x - 1;
  if (copier) {
    stage_to_w<T, PB>(w, ld, copy_j0, copy_n, copy);
    return;
  }
  potrf_panel<T, PB>(sm, w, ld, j0, n, k, info, stage, blockIdx.x, gridDim.x - (copy != nullptr ? 1 : 0));
}

template <typename T, int PB>
__global__ __launch_bounds__(256) void stage_to_w_kernel(T* __restrict__ w, int64_t ld, int64_t j0, int n,
                                                         const T* __restrict__ stage) {
  stage_to_w<T, PB>(w, ld, j0, n, stage);
}

// fp64 left-looking update of a panel's columns from its strip's earlier panels (the one-panel-per-launch
// Cholesky's narrow product): D = W[j0:, j0:j0+n] -= W[j0:, s0:j0] W[j0:j0+n, s0:j0]^T, on D's lower triangle,
// with K = j0 - s0 = 32 NT.  One workgroup per 32 rows of D (M rows in all), wave w the 16 x 16 block
// (w / 2, w % 2) over the whole k range: every operand load issued at once, 128 bits at a time (rows contiguous
// along k, 16-byte aligned), then the MFMA chain (v_mfma_f64_16x16x4_f64) in the order of the LDS-direct
// strided GEMM's tiles -- lane (q, h) = (l % 16, l / 16) supplies A(q, k) and B(k, q) with k = 32 t + 8 h + 2 v + s2
// to MFMA (v, s2) of k-tile t -- then D - acc, so the result is that GEMM's bit for bit.  The GEMM takes a k-tile
// at a time through LDS behind a barrier each; this kernel waits out one memory latency for the whole product.
template <int NT>
__global__ __launch_bounds__(256) void narrow_update64_kernel(double* __restrict__ w, int64_t ld, int64_t j0,
                                                              int64_t s0, int64_t M, int n) {
  typedef double doublex4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 15, h = lane >> 4;
  const int64_t ib = (int64_t)blockIdx.x * 32 + 16 * (wave >> 1);  // the block's first row of D
  const int cb = 16 * (wave & 1);                                   // and first column
  const bool a_in = ib + q < M, b_in = cb + q < n;
  const double* ap = w + (j0 + (a_in ? ib + q : 0)) * ld + s0 + 8 * h;
  const double* bp = w + (j0 + (b_in ? cb + q : 0)) * ld + s0 + 8 * h;
  double2 av[NT][4], bv[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      av[t][v] = a_in ? *reinterpret_cast<const double2*>(ap + 32 * t + 2 * v) : double2{0., 0.};
      bv[t][v] = b_in ? *reinterpret_cast<const double2*>(bp + 32 * t + 2 * v) : double2{0., 0.};
    }
  doublex4 acc = {0., 0., 0., 0.};
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[t][v].x, bv[t][v].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[t][v].y, bv[t][v].y, acc, 0, 0, 0);
    }
  // accumulator element r: D(ib + h + 4 r, cb + q); the loads of D first, then the stores
  const int c = cb + q;
  double old[4];
  bool ok[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int64_t i = ib + h + 4 * r;
    ok[r] = i < M && c < n && c <= i;
    old[r] = ok[r] ? w[(j0 + i) * ld + j0 + c] : 0.;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    old[r] = old[r] - acc[r];
    asm volatile("" : "+v"(old[r]));  // computed before the stores' branches
  }
#pragma unroll
  for (int r = 0; r < 4; ++r)
    if (ok[r]) w[(j0 + ib + h + 4 * r) * ld + j0 + c] = old[r];
}

// One wave per diagonal NB block of the lower triangular W: replace it by its inverse.
template <typename T, int NB>
__global__ __launch_bounds__(64) void trtri_leaf_kernel(T* __restrict__ w, int64_t ld, int64_t k, int64_t mstride) {
  w += (int64_t)blockIdx.y * mstride;  // matrix blockIdx.y of a group
  const int lane = threadIdx.x;
  const int64_t b0 = (int64_t)blockIdx.x * NB;
  const int n = k - b0 < NB ? (int)(k - b0) : NB;
  T a[NB], x[NB];
  T* row = w + (b0 + lane) * ld + b0;
#pragma unroll
  for (int c = 0; c < NB; ++c) a[c] = (lane < n && c <= lane) ? row[c] : (c == lane ? T(1) : T(0));
  wave_trtri<T, NB>(a, x, lane);
  if (lane < n) {
#pragma unroll
    for (int c = 0; c < NB; ++c)
      if (c <= lane && c < n) row[c] = x[c];
  }
}

// L(i, j) from L_raw(i, j) = w[base + i*rs + j*cs]: L_raw(i,j)/L_raw(j,j) below the diagonal,
// 1 on it, 0 above.  32 x 32 tiles through LDS so that both the read and the write coalesce.
template <typename T>
__global__ __launch_bounds__(256) void normalize_unit_kernel(T* __restrict__ out, const T* __restrict__ w,
                                                             int64_t k, int64_t base, int64_t rs, int64_t cs, int64_t mstride) {
  out += (int64_t)blockIdx.z * mstride;  // matrix blockIdx.z of a group
  w += (int64_t)blockIdx.z * mstride;
  __shared__ T tile[32][33];
  __shared__ T diag[32];
  const int64_t i0 = (int64_t)blockIdx.y * 32, j0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  const bool row_fast = rs == 1 || rs == -1;  // w contiguous along i: threads run along i to load
  if (j0 <= i0 + 31) {
    for (int yy = ty; yy < 32; yy += 8) {
      const int li = row_fast ? tx : yy, lj = row_fast ? yy : tx;
      const int64_t i = i0 + li, j = j0 + lj;
      tile[li][lj] = (i < k && j < k && j < i) ? w[base + i * rs + j * cs] : T(0);
    }
    if (threadIdx.x < 32) {
      const int64_t j = j0 + threadIdx.x;
      diag[threadIdx.x] = j < k ? w[base + j * rs + j * cs] : T(1);
    }
  }
  __syncthreads();
  for (int yy = ty; yy < 32; yy += 8) {
    const int64_t i = i0 + yy, j = j0 + tx;
    if (i >= k || j >= k) continue;
    T v = T(0);
    if (j == i) v = T(1);
    else if (j < i) v = tile[yy][tx] / diag[tx];
    out[i * k + j] = v;
  }
}

// U = L^T for unit (size 1) normalisation: U(i, j) = L_raw(j, i) / L_raw(i, i) above the diagonal, 1 on it, 0
// below -- the same quotients as L(j, i), so U is L's transpose bit for bit.  L_raw(j, i) = w[base + j rs + i cs]
// runs along j with stride rs (the reversed copy of ldl_of_inverse: rs = -1), so threads along j read and write
// contiguously without an LDS transpose.
template <typename T>
__global__ __launch_bounds__(256) void normalize_unit_upper_kernel(T* __restrict__ out, const T* __restrict__ w,
                                                                   int64_t k, int64_t base, int64_t rs, int64_t cs,
                                                                   int64_t mstride) {
  out += (int64_t)blockIdx.z * mstride;
  w += (int64_t)blockIdx.z * mstride;
  __shared__ T diag[32];
  const int64_t i0 = (int64_t)blockIdx.y * 32, j0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  if (threadIdx.x < 32) {
    const int64_t i = i0 + threadIdx.x;
    diag[threadIdx.x] = i < k ? w[base + i * rs + i * cs] : T(1);
  }
  __syncthreads();
  for (int yy = ty; yy < 32; yy += 8) {
    const int64_t i = i0 + yy, j = j0 + tx;
    if (i >= k || j >= k) continue;
    T v = T(0);
    if (j == i) v = T(1);
    else if (j > i) v = w[base + j * rs + i * cs] / diag[yy];
    out[i * k + j] = v;
  }
}

// Block normalisation for p x p blocks (p <= NB): a workgroup owns column block b and 64 rows.
// Rows below the block get L_raw(i, block) D_b^{-1}; the block itself becomes I; rows above, 0.
template <typename T, int NB>
__global__ __launch_bounds__(256) void normalize_block_kernel(T* __restrict__ out, const T* __restrict__ w,
                                                              int64_t k, int p, int64_t base, int64_t rs,
                                                              int64_t cs, int64_t mstride) {
  out += (int64_t)blockIdx.z * mstride;  // matrix blockIdx.z of a group
  w += (int64_t)blockIdx.z * mstride;
  __shared__ T dinv[NB][NB + 1];
  __shared__ T rows[64][NB + 1];
  const int64_t b = blockIdx.x, c0 = b * p;
  const int64_t i0 = (int64_t)blockIdx.y * 64;
  const int tid = threadIdx.x;
  const bool below = i0 + 63 >= c0 + p;  // this chunk has rows strictly below the block
  if (below) {
    if (tid < 64) {
      const int lane = tid;
      T a[NB], x[NB];
#pragma unroll
      for (int c = 0; c < NB; ++c)
        a[c] = (lane < p && c < p && c <= lane) ? w[base + (c0 + lane) * rs + (c0 + c) * cs]
                                                : (c == lane ? T(1) : T(0));
      wave_trtri<T, NB>(a, x, lane);
      if (lane < NB) {
#pragma unroll
        for (int c = 0; c < NB; ++c) dinv[lane][c] = x[c];
      }
    }
    for (int t = tid; t < 64 * p; t += 256) {
      const bool row_fast = rs == 1 || rs == -1;
      const int li = row_fast ? t % 64 : t / p, lc = row_fast ? t / 64 : t % p;
      const int64_t i = i0 + li;
      rows[li][lc] = (i < k && i >= c0 + p) ? w[base + i * rs + (c0 + lc) * cs] : T(0);
    }
  }
  __syncthreads();
  for (int t = tid; t < 64 * p; t += 256) {
    const int li = t / p, lc = t % p;
    const int64_t i = i0 + li, j = c0 + lc;
    if (i >= k) continue;
    T v;
    if (i < c0) {
      v = T(0);
    } else if (i < c0 + p) {
      v = (i - c0 == lc) ? T(1) : T(0);
    } else {
      v = T(0);
      for (int tt = lc; tt < p; ++tt) v += rows[li][tt] * dinv[tt][lc];
    }
    out[i * k + j] = v;
  }
}

// Block normalisation for NB < p <= PM: as normalize_block_kernel, but the rows below the block solve
// X D_b = R_b (forward substitution from the last column, one thread per row) against the diagonal block
// D_b staged in LDS, instead of multiplying by an inverse held in one wave's registers.
template <typename T, int PM>
__global__ __launch_bounds__(256) void normalize_block_solve_kernel(T* __restrict__ out, const T* __restrict__ w,
                                                                    int64_t k, int p, int64_t base, int64_t rs,
                                                                    int64_t cs, int64_t mstride) {
  out += (int64_t)blockIdx.z * mstride;  // matrix blockIdx.z of a group
  w += (int64_t)blockIdx.z * mstride;
  __shared__ T dblk[PM][PM + 1];
  __shared__ T rows[64][PM + 1];
  const int64_t b = blockIdx.x, c0 = b * p;
  const int64_t i0 = (int64_t)blockIdx.y * 64;
  const int tid = threadIdx.x;
  const bool below = i0 + 63 >= c0 + p;  // this chunk has rows strictly below the block
  const bool row_fast = rs == 1 || rs == -1;
  if (below) {
    for (int t = tid; t < p * p; t += 256) {
      const int r = row_fast ? t % p : t / p, cc = row_fast ? t / p : t % p;
      dblk[r][cc] = cc <= r ? w[base + (c0 + r) * rs + (c0 + cc) * cs] : T(0);
    }
    for (int t = tid; t < 64 * p; t += 256) {
      const int li = row_fast ? t % 64 : t / p, lc = row_fast ? t / 64 : t % p;
      const int64_t i = i0 + li;
      rows[li][lc] = (i < k && i >= c0 + p) ? w[base + i * rs + (c0 + lc) * cs] : T(0);
    }
  }
  __syncthreads();
  if (below && tid < 64) {
    const int64_t i = i0 + tid;
    if (i < k && i >= c0 + p) {
      T* x = rows[tid];
      for (int cc = p - 1; cc >= 0; --cc) {
        T acc = x[cc];
        for (int t = cc + 1; t < p; ++t) acc -= x[t] * dblk[t][cc];
        x[cc] = acc / dblk[cc][cc];
      }
    }
  }
  __syncthreads();
  for (int t = tid; t < 64 * p; t += 256) {
    const int li = t / p, lc = t % p;
    const int64_t i = i0 + li, j = c0 + lc;
    if (i >= k) continue;
    T v;
    if (i < c0)
      v = T(0);
    else if (i < c0 + p)
      v = (i - c0 == lc) ? T(1) : T(0);
    else
      v = rows[li][lc];
    out[i * k + j] = v;
  }
}

// Rank-K update of a lower trapezoid on fp32 MFMA (v_mfma_f32_32x32x2_f32):
//   D -= P P^T  on  D = W[r0.., r0..] (R x R; lower triangle, columns < C),  P = W[r0.., pc .. pc + K)
// with K a multiple of 32.  One workgroup per 128 x 128 block (bi, bj), four waves of 64 x 64 (2 x 2
// MFMA blocks each).  The K loop walks k-tiles of 32: both panels of a k-tile (the block's 128 rows
// of P, and the 128 rows that are its columns) are loaded one k-tile ahead straight into LDS
// (buffer loads with the LDS destination bit), double-buffered, one barrier per k-tile; rows past R
// (A) or past min(R, C) (B) load as zeros.  Both panels use the same layout -- P's k runs along a row
// for both operands of D = P P^T: float f of a panel holds row f / 32 and k = 4 (q ^ quad_swizzle(row))
// + f % 4, q = (f % 32) / 4 (16-byte k-quads XOR-swizzled by row, lds_dma.h, so that the lanes reading one
// quad of different rows hit different bank groups), and every fragment read is 128 bits.  Lane l (i = l % 32, h = l / 32)
// feeds A(i, 16 h + s) and B(16 h + s, i) to MFMA s; the accumulators hold
// D(8 (r / 4) + 4 h + r % 4, i).  The epilogue subtracts the products from D in place (read all
// 16 entries of a block, then write), masked to the lower triangle, to i < R and to j < C.
//
// The same kernel serves the three updates of the two-level Cholesky below: a panel's update of the
// next panel's columns (C = 64), its update of the rest of its strip (rank 64), and a strip's update of the
// whole trailing triangle (rank 512 or 1024).
constexpr int WB = 128;  // block edge
constexpr int WK = 32;   // k-tile depth

struct WideLds {
  float a[2][WB * WK];
  float b[2][WB * WK];
};

__device__ __forceinline__ void syrk_wide_block(WideLds& sm, float* __restrict__ w, int64_t ld, int64_t r0, int R,
                                                int C, int64_t pc, int K, int bi, int bj) {
  const int tid = threadIdx.x, lane = tid & 63, li = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wy = wave >> 1, wx = wave & 1;
  const int I0 = bi * WB, J0 = bj * WB;
  const int ild = (int)ld;
  const int CR = C < R ? C : R;
  // the panels' buffer resources are based at the block's own first rows (A: rows r0 + I0 .., B: rows
  // r0 + J0 ..), so that every byte offset stays below 128 rows of ld floats at any matrix size
  const int arows = R - I0 < WB ? R - I0 : WB, brows = CR - J0 < WB ? CR - J0 : WB;
  const __amdgpu_buffer_rsrc_t rpa =
      matrix_rsrc(w + (r0 + I0) * ld + pc, arows > 0 ? (int64_t)(arows - 1) * ld + K : 0);
  const __amdgpu_buffer_rsrc_t rpb =
      matrix_rsrc(w + (r0 + J0) * ld + pc, brows > 0 ? (int64_t)(brows - 1) * ld + K : 0);

  // per-lane staging offsets of the wave's four 128-bit loads per panel and k-tile
  int aoff[4], boff[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int f = (wave + 4 * x) * 256 + 4 * lane;
    const int row = f >> 5, kq = ((f >> 2) & 7) ^ quad_swizzle(row);
    aoff[x] = row < arows ? (row * ild + 4 * kq) * 4 : OOB;
    boff[x] = row < brows ? (row * ild + 4 * kq) * 4 : OOB;
  }
  // a block whose rows and columns all lie inside the update takes the k offset in the loads' scalar field:
  // no vector instruction beside the MFMA bursts
  const bool full = I0 + WB <= R && J0 + WB <= CR;
  auto issue = [&](int t, int buf) {
    if (full) {
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int f0 = (wave + 4 * x) * 256;
        dma_load_so<4>(rpa, &sm.a[buf][f0], aoff[x], t * WK * 4);
        dma_load_so<4>(rpb, &sm.b[buf][f0], boff[x], t * WK * 4);
      }
      return;
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int f0 = (wave + 4 * x) * 256;
      dma_load<4>(rpa, &sm.a[buf][f0], aoff[x] == OOB ? OOB : aoff[x] + t * WK * 4);
      dma_load<4>(rpb, &sm.b[buf][f0], boff[x] == OOB ? OOB : boff[x] + t * WK * 4);
    }
  };

  // a wave with nothing to write (above the diagonal, right of C or below R) still loads and waits
  const bool act = !(bi == bj && wy < wx) && J0 + 64 * wx < C && I0 + 64 * wy < R;
  floatx16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][d][r] = 0.f;

  const int sw = quad_swizzle(li);
  const int a_base = (64 * wy + li) * WK, b_base = (64 * wx + li) * WK;
  auto step = [&](int t, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    __syncthreads();  // buffer cur is complete; buffer 1 - cur is no longer read
    if (t + 1 < K / WK) issue(t + 1, 1 - cur);
    if (act) {
      const float* as = &sm.a[cur][a_base];
      const float* bs = &sm.b[cur][b_base];
      float4 fa[2][2], fb[2][2];
      auto frag = [&](int v, int slot) {
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          fa[slot][a] = *reinterpret_cast<const float4*>(as + a * 32 * WK + 4 * ((4 * hh + v) ^ sw));
          fb[slot][a] = *reinterpret_cast<const float4*>(bs + a * 32 * WK + 4 * ((4 * hh + v) ^ sw));
        }
      };
      frag(0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (v < 3) frag(v + 1, (v + 1) & 1);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
          for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int d = 0; d < 2; ++d)
              acc[a][d] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[v & 1][a][s2], fb[v & 1][d][s2], acc[a][d], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_dma();  // this wave's loads of k-tile t + 1 have landed before the next barrier
  };
  issue(0, 0);
  wait_dma();
  for (int t = 0; t < K / WK; t += 2) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < K / WK) step(t + 1, std::integral_constant<int, 1>{});
  }
  if (!act) return;
  // the block of D at rows r0 + I0 .., columns r0 + J0 .. (a resource based there: offsets below 128 rows)
  const __amdgpu_buffer_rsrc_t rd = matrix_rsrc(w + (r0 + I0) * ld + r0 + J0, (int64_t)(arows - 1) * ld + WB);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      int off[16];
      float cur[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = I0 + 64 * wy + 32 * a + 8 * (r >> 2) + 4 * hh + (r & 3), j = J0 + 64 * wx + 32 * d + li;
        off[r] = (i < R && j < C && j <= i) ? ((i - I0) * ild + (j - J0)) * 4 : OOB;
        cur[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, off[r], 0, 0));
      }
#pragma unroll
      for (int r = 0; r < 16; ++r)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, cur[r] - acc[a][d][r]), rd, off[r], 0, 0);
    }
}

// Workgroup lin of n renumbered so that each XCD (own L2) runs a contiguous share of the blocks: the
// hardware deals workgroup w to XCD w % 8.
__device__ __forceinline__ int64_t xcd_contiguous(int64_t lin, int64_t n) {
  const int64_t base = n / 8, extra = n % 8, xcd = lin % 8;
  return xcd * base + (xcd < extra ? xcd : extra) + lin / 8;
}

// Block (bi, bj) number id of a lower trapezoid of blocks with nbc block columns, numbered row by
// row: the triangle of the first nbc block rows, then nbc blocks per row.
__device__ __forceinline__ void trapezoid_block(int64_t id, int64_t nbc, int& bi, int& bj) {
  const int64_t tri = nbc * (nbc + 1) / 2;
  if (id >= tri) {
    bi = (int)(nbc + (id - tri) / nbc);
    bj = (int)((id - tri) % nbc);
    return;
  }
  int64_t ti = (int64_t)((sqrt(8.0 * (double)id + 1.0) - 1.0) * 0.5);
  while ((ti + 1) * (ti + 2) / 2 <= id) ++ti;
  while (ti * (ti + 1) / 2 > id) --ti;
  bi = (int)ti;
  bj = (int)(id - ti * (ti + 1) / 2);
}

// Workgroups of a trapezoid update (R x R lower triangle, columns < C; C <= R).
__host__ __device__ inline int64_t trapezoid_blocks(int64_t R, int64_t C) {
  const int64_t nb = (R + WB - 1) / WB, nbc = (C + WB - 1) / WB;
  return nbc * (nbc + 1) / 2 + (nb - nbc) * nbc;
}

// A panel's update of the next panel's columns (D's first PB columns, every row: blocks (x, 0));
// the last workgroup copies the staged diagonal block of panel `sc` (PB rows) into W.
// The matrix of a launch of the fp32 Cholesky (blockIdx.y selects one of a group, see CholeskyRun):
// W, its info word, the staging block of the launch's panel and the staged block to copy into W
// (nullptr: none).
struct PanelPtrs {
  float* w;
  int* info;
  float* stage;
  const float* copy;
};

// Matrices of one size factored by the same launches (entries [0, gridDim.y) used), passed by value.
constexpr int GROUP_MAX = 16;
struct PanelGroup {
  PanelPtrs p[GROUP_MAX];
};

template <int PB>
__global__ __launch_bounds__(256, 2) void syrk_strip_kernel(PanelGroup grp, int64_t ld, int64_t r0, int R,
                                                            int64_t pc, int K, int64_t sc) {
  __shared__ __align__(16) WideLds sm;
  const PanelPtrs& p = grp.p[blockIdx.y];
  if (blockIdx.x == gridDim.x - 1) {
    stage_to_w<float, PB>(p.w, ld, sc, PB, p.stage);
    return;
  }
  syrk_wide_block(sm, p.w, ld, r0, R, PB, pc, K, (int)blockIdx.x, 0);
}

// Look-ahead step of the fp32 Cholesky: workgroups [0, n_potrf) factor and solve panel j0; the
// others apply a pending trapezoid update (square W[r0.., r0..], R x R, columns < C, rank K from
// P = W[r0.., pc .. pc + K)).  The two touch disjoint columns, so the panel's latency-bound
// factorisation runs beside the throughput-bound update.
// upc >= 0: the panel first takes the rank-PB update of the panel at columns [upc, upc + PB) itself.
// copy != nullptr: the last workgroup moves that earlier panel's staged diagonal block (at column
// copy_j0, PB rows) into W.  The matrix: entry blockIdx.y of the group (the copy set in all or none).
template <int PB>
__global__ __launch_bounds__(256, 2) void panel_step_kernel(PanelGroup grp, int64_t ld, int64_t j0, int n, int64_t k,
                                                            int64_t n_potrf, int64_t r0, int R, int C, int64_t pc,
                                                            int K, int64_t upc, int64_t copy_j0) {
  __shared__ __align__(16) union {
    PotrfLds<float, PB> p;
    WideLds s;
  } sm;
  const PanelPtrs& p = grp.p[blockIdx.y];
  const int64_t n_upd = gridDim.x - n_potrf - (p.copy ? 1 : 0);
  if (p.copy && (int64_t)blockIdx.x == gridDim.x - 1) {
    stage_to_w<float, PB>(p.w, ld, copy_j0, PB, p.copy);
    return;
  }
  if ((int64_t)blockIdx.x < n_potrf) {
    potrf_panel<float, PB>(sm.p, p.w, ld, j0, n, k, p.info, p.stage, blockIdx.x, n_potrf, upc);
    return;
  }
  int bi, bj;
  trapezoid_block(xcd_contiguous(blockIdx.x - n_potrf, n_upd), (C + WB - 1) / WB, bi, bj);
  syrk_wide_block(sm.s, p.w, ld, r0, R, C, pc, K, bi, bj);
}

// Launch sequence of the blocked Cholesky of W (k x k) in place over the panels [col_begin, col_end)
// (multiples of PB; col_end < 0: to the end), one panel per step() so that one host thread can
// interleave two factorisations on two streams.  Between runs (and after finish()) every factored
// diagonal block is in W; between two steps of a run the fp64 path may still hold the last panel's block in
// its staging slot (the next panel's launch moves it).  Two-level fp32 path: every earlier panel's update has been applied to the
// whole trailing matrix (finish() issues a pending one).  Plain path (fp64, fp32 with k % 4 != 0): the
// panels of the strip [j0 / NS * NS, j0) have updated nothing to their right yet -- a later panel of the
// strip takes them by its left-looking update and the strip's end by its rank-NS update, both reading
// W[:, strip start : j0] -- so ranges must be run in column order, as the single call runs them, and
// then issue the single call's launches in its order.  stage: PB x PB elements of scratch (a panel's factored diagonal block between its
// launch and the next).  twin() (two-level path only): up to GROUP_MAX - 1 more k x k matrices factored
// by the same launches, as blockIdx.y = 1, 2, ... of each -- one chain of latency-bound panel launches for
// all, and the work of all in each throughput-bound update; each matrix sees the launches it would see
// alone.
template <typename T>
struct CholeskyRun {
  static constexpr int PB = LdlBlock<T>::PB;
  // strip width of the two-level fp32 path: 1024 columns from k = 8192, 512 below (both 8192 factors 10.53 ms
  // with 256, 10.32 with 512, 10.16-10.25 with 1024; 14336 + 4096: 23.14 with 512, 22.72-22.90 with 1024; 4096:
  // 3.15 with 256, 3.12 with 512, 3.22 with 1024).  The inverse's split points (multiples of 1024,
  // trtri_split) must be strip boundaries: the strip launch of the panel before one copies that panel's
  // diagonal block into W, which the inverse's first part reads from beside the rest of the chain.
  static constexpr int64_t SW_SMALL = 8 * PB, SW_LARGE = 16 * PB;
  static_assert(1024 % SW_SMALL == 0 && 1024 % SW_LARGE == 0, "every split point of the inverse is a strip boundary");
  T* w;
  int64_t k;
  int* info;
  T* stage;
  hipStream_t stream;
  int64_t col_begin, col_end, j0;
  int64_t sw;  // strip width (two-level path)
  bool two_level, fuse, fold, done = false;
  int64_t pr0 = 0, pC = 0, ppc = 0;  // pending trapezoid update (columns < pC of W[pr0.., pr0..])
  int64_t pend_j0 = -1;              // plain path: a panel whose staged block is not in W yet (or -1)
  int pend_n = 0;
  int pK = 0;
  int ng = 1;  // matrices of the group; entry 0 is (w, info, stage)
  T* wg[GROUP_MAX] = {};
  int* infog[GROUP_MAX] = {};
  T* stageg[GROUP_MAX] = {};

  CholeskyRun(T* w_, int64_t k_, int* info_, T* stage_, hipStream_t s, int64_t cb = 0, int64_t ce = -1)
      : w(w_), k(k_), info(info_), stage(stage_), stream(s), col_begin(cb), col_end(ce < 0 || ce > k_ ? k_ : ce),
        j0(cb) {
    // (the update kernels' offsets are relative to their blocks' rows: 128 ld floats, any k below 2^22)
    two_level = sizeof(T) == 4 && k % 4 == 0 && k < ((int64_t)1 << 22);
    sw = k >= 8192 ? SW_LARGE : SW_SMALL;
    fuse = two_level && k * k >= 2 * (int64_t)PB * PB;
    // fp64 with two staging slots: a panel's block moves into W in the next panel's launch.  The factor pair's
    // inverse reads the leading columns from W beside the rest of the chain as soon as the chain has passed them
    // (trtri_split): it moves the last of those blocks first (flush_staged).  Not in fp32, whose two-level path
    // copies each strip's last block in its strip launch.
    fold = sizeof(T) == 8 && !two_level && k * k >= 2 * (int64_t)PB * PB;
    done = j0 >= col_end;
    wg[0] = w_;
    infog[0] = info_;
    stageg[0] = stage_;
  }

  // Factor one more matrix (same k, its own info word and staging blocks) in the same launches; false
  // (nothing changed) off the two-level path, with a full group or once a step was taken.
  bool twin(T* w_, int* info_, T* stage_) {
    if (!two_level || j0 != col_begin || done || ng == GROUP_MAX) return false;
    wg[ng] = w_;
    infog[ng] = info_;
    stageg[ng] = stage_;
    ++ng;
    return true;
  }

  // Staging block of panel j of matrix f (two alternating ones when fused or folded: a panel's launch copies
  // the previous panel's block into W while its own workgroups stage the new one).
  T* slot(int64_t j, int f = 0) const {
    T* st = stageg[f];
    return (fuse || fold) && ((j / PB) & 1) ? st + (int64_t)PB * PB : st;
  }

  // The launches of panel j0, then j0 += PB.
  int step() {
    if (done) return 0;
    int rc;
    if constexpr (sizeof(T) == 4)
      rc = two_level ? step_two_level() : step_plain();
    else
      rc = step_plain();
    if (rc) return rc;
    j0 += PB;
    if (!done && j0 >= col_end) {
      done = true;
      return finish();
    }
    return 0;
  }

  // The pending staged block (fold) into W now, with no launch of its own left to wait for it.
  int flush_staged() {
    if (pend_j0 < 0) return 0;
    hipLaunchKernelGGL((stage_to_w_kernel<T, PB>), dim3(1), dim3(256), 0, stream, w, k, pend_j0, pend_n,
                       (const T*)slot(pend_j0));
    pend_j0 = -1;
    return (int)hipGetLastError();
  }

 private:
  // fp32, two levels: strips of sw columns (aligned to multiples of sw, cut at the range ends).
  // Inside a strip, each panel updates only the strip's later columns (rank PB); after a strip's
  // last panel, one rank-(strip width) update covers everything to its right -- four times the
  // arithmetic per byte of the trailing triangle that a rank-PB update moves.  Look-ahead: the
  // update of the next panel's columns runs on its own (strip kernel), the rest of the update runs
  // in the launch that factors the next panel.
  int step_two_level() {
    int rc;
    const int n = k - j0 < PB ? (int)(k - j0) : PB;
    const int64_t rest = k - j0 - PB;
    const int64_t blocks = rest > 0 ? (cdiv(rest, 64) < 256 ? cdiv(rest, 64) : 256) : 1;
    const int64_t pR = pC > 0 ? k - pr0 : 0;
    const int64_t upd = pC > 0 ? trapezoid_blocks(pR, pC) : 0;
    // the strip of panel j0: [s_lo, s_hi)
    const int64_t s_al = j0 / sw * sw;
    const int64_t s_lo = s_al > col_begin ? s_al : col_begin;
    const int64_t s_hi = s_al + sw < col_end ? s_al + sw : col_end;
    // fused: a panel after the first of its strip takes the previous panel's rank-PB update itself
    // (no launch of its own for it), and its launch moves the previous panel's staged block into W
    const bool in_strip = fuse && j0 > s_lo;
    const unsigned ny = (unsigned)ng;
    PanelGroup pp{};
    for (int f = 0; f < ng; ++f)
      pp.p[f] = PanelPtrs{(float*)wg[f], infog[f], (float*)slot(j0, f),
                          in_strip ? (const float*)slot(j0 - PB, f) : nullptr};
    hipLaunchKernelGGL((panel_step_kernel<PB>), dim3((unsigned)(blocks + upd + (in_strip ? 1 : 0)), ny), dim3(256), 0,
                       stream, pp, k, j0, n, k, blocks, pr0, (int)pR, (int)pC, ppc, pK,
                       in_strip ? j0 - PB : (int64_t)-1, j0 - PB);
    if ((rc = (int)hipGetLastError())) return rc;
    pC = 0;
    if (rest <= 0) {  // the last panel: its staged block into W on its own
      for (unsigned f = 0; f < ny; ++f) {
        hipLaunchKernelGGL((stage_to_w_kernel<float, PB>), dim3(1), dim3(256), 0, stream, pp.p[f].w, k, j0, n,
                           (const float*)pp.p[f].stage);
        if ((rc = (int)hipGetLastError())) return rc;
      }
      done = true;
      return 0;
    }
    const bool strip_end = j0 + PB >= s_hi;
    // the update's rank: panel j0 alone inside the strip, the whole strip at its end
    const int64_t pc = strip_end ? s_lo : j0;
    const int K = (int)(j0 + PB - pc);
    if (strip_end || !fuse) {
      hipLaunchKernelGGL((syrk_strip_kernel<PB>), dim3((unsigned)cdiv(rest, WB) + 1, ny), dim3(256), 0, stream, pp, k,
                         j0 + PB, (int)rest, pc, K, j0);
      if ((rc = (int)hipGetLastError())) return rc;
    }
    // the rest: the strip's later columns, or everything to the right at a strip's end
    const int64_t r0 = j0 + 2 * PB, R = rest - PB;
    const int64_t C = strip_end ? R : (s_hi - r0 < R ? s_hi - r0 : R);
    if (R > 0 && C > 0) {
      pr0 = r0;
      pC = C;
      ppc = pc;
      pK = K;
    }
    return 0;
  }

  // fp64 (and fp32 with k % 4 != 0): strips of NS columns, left-looking inside a strip, right-looking
  // between strips.  Step j0: the panel's columns first receive the updates of the strip's earlier panels
  // (W[j0:, j0:j0+n] -= W[j0:, s0:j0] W[j0:j0+n, s0:j0]^T), then the panel is factored and its diagonal
  // block staged into W; at a strip's end the whole trailing triangle receives the strip in one rank-NS
  // update.  Against a rank-PB update of the trailing triangle per panel this reads and writes it once per
  // strip instead of once per panel (the update is bound by that traffic, not by its flops).
  static constexpr int64_t NS = 256;
  static_assert(NS % PB == 0, "strips hold whole panels");
  static_assert(sizeof(T) != 8 || (NS - PB) / 32 <= 7, "the fp64 narrow product's k-tiles: narrow_update64_kernel<1..7>");

  int step_plain() {
    int rc;
    const int n = k - j0 < PB ? (int)(k - j0) : PB;
    const int64_t rest = k - j0 - PB;
    const int64_t s0 = j0 / NS * NS;  // this panel's strip
    // fp64 with 16-byte aligned rows: the narrow product on its own kernel (the GEMM's bits, one memory
    // latency instead of one per k-tile)
    const bool narrow = sizeof(T) == 8 && k % 2 == 0 && ((uintptr_t)w & 15) == 0;
    if (j0 > s0 && narrow) {
      const int nt = (int)((j0 - s0) / 32);
      const dim3 grid((unsigned)cdiv(k - j0, 32));
      double* wd = reinterpret_cast<double*>(w);
      switch (nt) {
        case 1: hipLaunchKernelGGL(narrow_update64_kernel<1>, grid, dim3(256), 0, stream, wd, k, j0, s0, k - j0, n); break;
        case 2: hipLaunchKernelGGL(narrow_update64_kernel<2>, grid, dim3(256), 0, stream, wd, k, j0, s0, k - j0, n); break;
        case 3: hipLaunchKernelGGL(narrow_update64_kernel<3>, grid, dim3(256), 0, stream, wd, k, j0, s0, k - j0, n); break;
        case 4: hipLaunchKernelGGL(narrow_update64_kernel<4>, grid, dim3(256), 0, stream, wd, k, j0, s0, k - j0, n); break;
        case 5: hipLaunchKernelGGL(narrow_update64_kernel<5>, grid, dim3(256), 0, stream, wd, k, j0, s0, k - j0, n); break;
        case 6: hipLaunchKernelGGL(narrow_update64_kernel<6>, grid, dim3(256), 0, stream, wd, k, j0, s0, k - j0, n); break;
        case 7: hipLaunchKernelGGL(narrow_update64_kernel<7>, grid, dim3(256), 0, stream, wd, k, j0, s0, k - j0, n); break;
        default: return GPTQ2D_EINVAL;
      }
      if ((rc = (int)hipGetLastError())) return rc;
    } else if (j0 > s0) {
      GemmProblem<T> g{};
      g.M = k - j0;
      g.N = n;
      g.K = j0 - s0;
      g.batch = 1;
      g.A = w + j0 * k + s0;  // W[j0:, s0:j0]
      g.a_rs = k;
      g.a_cs = 1;
      g.B = g.A;  // B(kk, jj) = W[j0 + jj, s0 + kk]
      g.b_rs = 1;
      g.b_cs = k;
      g.D = w + j0 * k + j0;
      g.d_rs = k;
      g.d_cs = 1;
      g.alpha = T(-1);
      g.beta = T(1);
      g.d_tri = TRI_LOWER;
      if ((rc = gptq2d_gemm<T>(g, stream))) return rc;
    }
    const unsigned blocks = rest > 0 ? (unsigned)(cdiv(rest, 64) < 256 ? cdiv(rest, 64) : 256) : 1u;
    // the previous panel's staged block moves into W in this launch: no launch between the two panels reads
    // it (the updates read rows from the next panel's first on)
    const bool copy = pend_j0 >= 0;
    T* st = slot(j0);
    hipLaunchKernelGGL((potrf_panel_kernel<T, PB>), dim3(blocks + (copy ? 1u : 0u)), dim3(256), 0, stream, w, k, j0,
                       n, k, info, st, copy ? (const T*)slot(pend_j0) : nullptr, pend_j0, pend_n);
    if ((rc = (int)hipGetLastError())) return rc;
    pend_j0 = -1;
    if (rest <= 0 || !fold) {  // the last panel, or one staging slot: the block into W on its own
      hipLaunchKernelGGL((stage_to_w_kernel<T, PB>), dim3(1), dim3(256), 0, stream, w, k, j0, n, (const T*)st);
      if ((rc = (int)hipGetLastError())) return rc;
      if (rest <= 0) {
        done = true;
        return 0;
      }
    } else {
      pend_j0 = j0;
      pend_n = n;
    }
    const int64_t s1 = j0 + PB;
    if (s1 % NS) return 0;  // the strip goes on
    // trailing lower triangle: W22 -= P P^T with P = W[s1:, s0:s1]
    GemmProblem<T> g{};
    g.M = g.N = rest;
    g.K = s1 - s0;
    g.batch = 1;
    g.A = w + s1 * k + s0;
    g.a_rs = k;
    g.a_cs = 1;
    g.B = g.A;
    g.b_rs = 1;
    g.b_cs = k;
    g.D = w + s1 * k + s1;
    g.d_rs = k;
    g.d_cs = 1;
    g.alpha = T(-1);
    g.beta = T(1);
    g.d_tri = TRI_LOWER;
    return gptq2d_gemm<T>(g, stream);
  }

  // A range that stops early: the pending update (or the pending staged block) on its own.
  int finish() {
    if (const int rc = flush_staged()) return rc;
    if constexpr (sizeof(T) == 4) {
      if (pC <= 0) return 0;
      const int64_t pR = k - pr0;
      PanelGroup pp{};
      for (int f = 0; f < ng; ++f) pp.p[f] = PanelPtrs{(float*)wg[f], infog[f], (float*)stageg[f], nullptr};
      hipLaunchKernelGGL((panel_step_kernel<PB>), dim3((unsigned)trapezoid_blocks(pR, pC), (unsigned)ng), dim3(256),
                         0, stream, pp, k, (int64_t)0, 0, k, (int64_t)0, pr0, (int)pR, (int)pC, ppc, pK, (int64_t)-1,
                         (int64_t)0);
      pC = 0;
      return (int)hipGetLastError();
    }
    return 0;
  }
};

template <typename T>
int cholesky_inplace(T* w, int64_t k, int* info, T* stage, hipStream_t stream, int64_t col_begin = 0,
                     int64_t col_end = -1) {
  CholeskyRun<T> run(w, k, info, stage, stream, col_begin, col_end);
  int rc;
  while (!run.done)
    if ((rc = run.step())) return rc;
  return 0;
}

// Elements from the start of `out` where the Cholesky stages its factored diagonal blocks: the
// buffer's last 2 PB x PB elements (two alternating blocks; one, at the start, for k^2 < 2 PB^2 --
// CholeskyRun then does not fuse), away from what the triangular inverse's first part writes while
// the factorisation still runs.
template <typename T>
int64_t stage_offset(int64_t k) {
  constexpr int64_t PB = LdlBlock<T>::PB;
  return k * k >= 2 * PB * PB ? k * k - 2 * PB * PB : 0;
}

// Zero the strict upper triangle of the n x n diagonal block at w (row stride ld), one row per
// workgroup.
template <typename T>
__global__ __launch_bounds__(256) void zero_upper_kernel(T* __restrict__ w, int64_t ld, int64_t n, int64_t mstride) {
  w += (int64_t)blockIdx.y * mstride;  // matrix blockIdx.y of a group
  for (int64_t i = blockIdx.x; i < n; i += gridDim.x)
    for (int64_t j = i + 1 + threadIdx.x; j < n; j += 256) w[i * ld + j] = T(0);
}

// A level product of the triangular inverse, D = alpha A B (tri = 1: B lower, 2: A lower): the MFMA
// kernel that skips the zero triangle of the inverted block, or, where that kernel's layout
// conditions do not hold (rows not on 16-byte boundaries), the
// library's general strided GEMM with the same triangular structure.  (Sizes are not a condition: the MFMA
// kernel's buffer offsets are relative to its block's rows and to each k-tile's rows.)
int level_gemm(int64_t M, int64_t N, int64_t K, int64_t batch, const float* A, int64_t lda, int64_t sa,
               const float* B, int64_t ldb, int64_t sb, float* D, int64_t ldd, int64_t sd, float alpha, int tri,
               hipStream_t stream, int64_t ng = 1, int64_t mst = 0) {
  // ng problems of a group of matrices mst elements apart (A, B and D alike)
  TriGemm g{M, N, K, batch, A, lda, sa, B, ldb, sb, D, ldd, sd, alpha, tri, ng, mst, mst, mst};
  const int rc = gptq2d_tri_gemm_f32(g, stream);
  if (rc != GPTQ2D_EUNSUPPORTED) return rc;
  if (ng > 1) {
    for (int64_t z = 0; z < ng; ++z) {
      const int r = level_gemm(M, N, K, batch, A + z * mst, lda, sa, B + z * mst, ldb, sb, D + z * mst, ldd, sd, alpha,
                               tri, stream);
      if (r) return r;
    }
    return 0;
  }
  GemmProblem<float> h{};
  h.M = M;
  h.N = N;
  h.K = K;
  h.batch = batch;
  h.A = A;
  h.a_rs = lda;
  h.a_cs = 1;
  h.a_bs = sa;
  h.B = B;
  h.b_rs = ldb;
  h.b_cs = 1;
  h.b_bs = sb;
  h.D = D;
  h.d_rs = ldd;
  h.d_cs = 1;
  h.d_bs = sd;
  h.alpha = alpha;
  h.beta = 0.f;
  h.a_tri = tri == 2 ? TRI_LOWER : TRI_NONE;
  h.b_tri = tri == 1 ? TRI_LOWER : TRI_NONE;
  return gptq2d_gemm<float>(h, stream);
}

// In-place inverse of the lower triangular n x n diagonal block at w (row stride ld): leaves, then
// the levels.  tmp: >= n*n/4 + n elements for the levels' products.  tri (fp32): the levels on
// level_gemm; the block's strict upper triangle is zeroed first (the MFMA kernel reads it as the
// padding of the triangles' boundary k-tiles).
template <typename T>
int trtri_block(T* w, int64_t ld, int64_t n, T* tmp, bool tri, hipStream_t stream, int64_t ng = 1, int64_t mst = 0) {
  constexpr int NB = LdlBlock<T>::NB;
  int rc;
  // a group of ng matrices mst elements apart (w and tmp alike): one launch per step on the fp32 MFMA
  // levels, one matrix after the other on the general GEMM
  if (ng > 1 && !(sizeof(T) == 4 && tri)) {
    for (int64_t z = 0; z < ng; ++z)
      if ((rc = trtri_block<T>(w + z * mst, ld, n, tmp + z * mst, tri, stream))) return rc;
    return 0;
  }
  hipLaunchKernelGGL((trtri_leaf_kernel<T, NB>), dim3((unsigned)cdiv(n, NB), (unsigned)ng), dim3(64), 0, stream, w, ld,
                     n, mst);
  if ((rc = (int)hipGetLastError())) return rc;
  if (tri) {
    hipLaunchKernelGGL(zero_upper_kernel<T>, dim3((unsigned)(n < 8192 ? n : 8192), (unsigned)ng), dim3(256), 0, stream,
                       w, ld, n, mst);
    if ((rc = (int)hipGetLastError())) return rc;
  }
  for (int64_t s = NB; s < n; s *= 2) {
    const int64_t full = n / (2 * s);          // pairs with two full s-blocks
    const int64_t tail_r1 = full * 2 * s + s;  // a last, short pair starts its D block here
    const int64_t tail = tail_r1 < n ? n - tail_r1 : 0;
    for (int part = 0; part < 2; ++part) {
      const int64_t pairs = part == 0 ? full : (tail > 0 ? 1 : 0);
      if (pairs == 0) continue;
      const int64_t r0 = part == 0 ? 0 : full * 2 * s;
      const int64_t s2 = part == 0 ? s : tail;
      const int64_t bs = 2 * s * ld + 2 * s;
      if constexpr (sizeof(T) == 4) {
        if (tri) {
          // T = B A^{-1}, then B <- -D^{-1} T
          if ((rc = level_gemm(s2, s, s, pairs, w + (r0 + s) * ld + r0, ld, bs, w + r0 * ld + r0, ld, bs, tmp, s,
                               s2 * s, 1.f, 1, stream, ng, mst)))
            return rc;
          if ((rc = level_gemm(s2, s, s2, pairs, w + (r0 + s) * ld + (r0 + s), ld, bs, tmp, s, s2 * s,
                               w + (r0 + s) * ld + r0, ld, bs, -1.f, 2, stream, ng, mst)))
            return rc;
          continue;
        }
      }
      // T = B A^{-1}: (s2 x s) = (s2 x s) (s x s, lower)
      GemmProblem<T> g{};
      g.M = s2;
      g.N = s;
      g.K = s;
      g.batch = pairs;
      g.A = w + (r0 + s) * ld + r0;  // B block
      g.a_rs = ld;
      g.a_cs = 1;
      g.a_bs = bs;
      g.B = w + r0 * ld + r0;  // A^{-1}
      g.b_rs = ld;
      g.b_cs = 1;
      g.b_bs = bs;
      g.b_tri = TRI_LOWER;
      g.D = tmp;
      g.d_rs = s;
      g.d_cs = 1;
      g.d_bs = s2 * s;
      g.alpha = T(1);
      g.beta = T(0);
      if ((rc = gptq2d_gemm<T>(g, stream))) return rc;
      // B <- -D^{-1} T: (s2 x s) = (s2 x s2, lower) (s2 x s)
      GemmProblem<T> h{};
      h.M = s2;
      h.N = s;
      h.K = s2;
      h.batch = pairs;
      h.A = w + (r0 + s) * ld + (r0 + s);  // D^{-1}
      h.a_rs = ld;
      h.a_cs = 1;
      h.a_bs = bs;
      h.a_tri = TRI_LOWER;
      h.B = tmp;
      h.b_rs = s;
      h.b_cs = 1;
      h.b_bs = s2 * s;
      h.D = w + (r0 + s) * ld + r0;
      h.d_rs = ld;
      h.d_cs = 1;
      h.d_bs = bs;
      h.alpha = T(-1);
      h.beta = T(0);
      if ((rc = gptq2d_gemm<T>(h, stream))) return rc;
    }
  }
  return 0;
}

// Split point of the triangular inverse of a k x k factor: s = NB 2^j, the largest below k, from k = 2048
// (fp32: levels on level_gemm; fp64: on the strided GEMM); 0: no split.  With a split, the inverse of C = [A 0; B D]
// (A: s x s) runs in three parts:
//   1. A^{-1} in place and T = B A^{-1} -- these read only the Cholesky's columns < s, so they can
//      run while the factorisation of the columns >= s goes on;
//   2. D^{-1} in place, once the factorisation is complete;
//   3. B <- -D^{-1} T, and the normalisation into out.
// The levels below s are the same whether or not the inverse is split (the recursive doubling pairs
// blocks aligned to multiples of their size, and s is a multiple of every lower level's pair size).
template <typename T>
int64_t trtri_split(int64_t k) {
  if (k < 2048) return 0;
  int64_t s = LdlBlock<T>::NB;
  while (2 * s < k) s *= 2;
  return s;
}

// Where the three parts keep their data in `out` (k x k elements, free until the normalisation; its
// last 2 PB x PB elements stage the Cholesky's diagonal blocks while part 1 runs): T (n2 x s, and
// before it part 1's level products), then part 2's level products -- disjoint, as parts 1 and 2
// may run at the same time.  s >= k / 2 >= n2, so n2 s + n2^2 / 4 + n2 stays below k^2 - 2 PB^2.
struct TrtriLayout {
  int64_t s, n2, t_off, tmp2_off;
};

template <typename T>
TrtriLayout trtri_layout(T* out, int64_t k, int64_t s) {
  TrtriLayout L{};
  L.s = s;
  L.n2 = k - s;
  L.t_off = 0;
  const int64_t t_end = L.n2 * s > s * s / 4 + s ? L.n2 * s : s * s / 4 + s;
  L.tmp2_off = t_end;
  return L;
}

// In-place inverse of the lower triangular W (k x k) in one sequence; tmp: a buffer of >= k*k/4 + k
// elements for the levels' products.  fp32 from k = 512: the levels on level_gemm.
template <typename T>
int trtri_inplace(T* w, int64_t k, T* tmp, hipStream_t stream, int64_t ng = 1, int64_t mst = 0) {
  return trtri_block<T>(w, k, k, tmp, sizeof(T) == 4 && k >= 512, stream, ng, mst);
}

template <typename T>
int normalize(T* out, const T* w, int64_t k, int64_t size, int64_t base, int64_t rs, int64_t cs, hipStream_t stream,
              int64_t ng = 1, int64_t mst = 0, bool upper = false);

// Part `phase` (1, 2, 3 as at trtri_split) of the inverse of the Cholesky factor in work and the
// normalisation into out (L_raw(i, j) = C^{-1}(k-1-j, k-1-i) = work[(k-1-j) k + (k-1-i)]).  Without
// a split, part 1 does nothing, part 2 is the whole inverse and part 3 the normalisation.  ng > 1: the
// same part of a group of ng matrices k^2 elements apart (out and w alike), in one launch per step.
template <typename T>
int trtri_part(T* out, T* w, int64_t k, int64_t size, int phase, hipStream_t stream, int64_t ng = 1,
               bool upper = false) {
  const int64_t s = trtri_split<T>(k), mst = k * k;
  int rc = 0;
  if (s == 0) {
    if (phase == 2) return trtri_inplace<T>(w, k, out, stream, ng, mst);
    if (phase == 3) return normalize<T>(out, w, k, size, (k - 1) * k + (k - 1), -1, -k, stream, ng, mst, upper);
    return 0;
  }
  const TrtriLayout L = trtri_layout<T>(out, k, s);
  if constexpr (sizeof(T) == 4) {
    if (phase == 1) {
      if ((rc = trtri_block<T>(w, k, s, out + L.t_off, true, stream, ng, mst))) return rc;
      // T = B A^{-1}: (n2 x s) = (n2 x s) (s x s)
      return level_gemm(L.n2, s, s, 1, w + s * k, k, 0, w, k, 0, out + L.t_off, s, 0, 1.f, 1, stream, ng, mst);
    }
    if (phase == 2) return trtri_block<T>(w + s * k + s, k, L.n2, out + L.tmp2_off, true, stream, ng, mst);
    if (phase == 3) {
      // B <- -D^{-1} T: (n2 x s) = (n2 x n2) (n2 x s)
      if ((rc = level_gemm(L.n2, s, L.n2, 1, w + s * k + s, k, 0, out + L.t_off, s, 0, w + s * k, k, 0, -1.f, 2,
                           stream, ng, mst)))
        return rc;
      return normalize<T>(out, w, k, size, (k - 1) * k + (k - 1), -1, -k, stream, ng, mst, upper);
    }
  } else {
    // fp64: the same parts on the strided GEMM -- the calls that trtri_inplace's levels make for these blocks
    // (its top level is this split's T and -D^{-1} T), so the same bits; a group one matrix after the other
    for (int64_t z = 0; z < ng; ++z) {
      T* wz = w + z * mst;
      T* tz = out + z * mst + L.t_off;
      if (phase == 1) {
        if ((rc = trtri_block<T>(wz, k, s, tz, false, stream))) return rc;
        GemmProblem<T> g{};  // T = B A^{-1}: (n2 x s) = (n2 x s) (s x s, lower)
        g.M = L.n2;
        g.N = s;
        g.K = s;
        g.batch = 1;
        g.A = wz + s * k;
        g.a_rs = k;
        g.a_cs = 1;
        g.B = wz;
        g.b_rs = k;
        g.b_cs = 1;
        g.b_tri = TRI_LOWER;
        g.D = tz;
        g.d_rs = s;
        g.d_cs = 1;
        g.alpha = T(1);
        g.beta = T(0);
        if ((rc = gptq2d_gemm<T>(g, stream))) return rc;
      } else if (phase == 2) {
        if ((rc = trtri_block<T>(wz + s * k + s, k, L.n2, out + z * mst + L.tmp2_off, false, stream))) return rc;
      } else if (phase == 3) {
        GemmProblem<T> h{};  // B <- -D^{-1} T: (n2 x s) = (n2 x n2, lower) (n2 x s)
        h.M = L.n2;
        h.N = s;
        h.K = L.n2;
        h.batch = 1;
        h.A = wz + s * k + s;
        h.a_rs = k;
        h.a_cs = 1;
        h.a_tri = TRI_LOWER;
        h.B = tz;
        h.b_rs = s;
        h.b_cs = 1;
        h.D = wz + s * k;
        h.d_rs = k;
        h.d_cs = 1;
        h.alpha = T(-1);
        h.beta = T(0);
        if ((rc = gptq2d_gemm<T>(h, stream))) return rc;
      }
    }
    if (phase == 3) return normalize<T>(out, w, k, size, (k - 1) * k + (k - 1), -1, -k, stream, ng, mst, upper);
  }
  return rc;
}

template <typename T>
int normalize(T* out, const T* w, int64_t k, int64_t size, int64_t base, int64_t rs, int64_t cs, hipStream_t stream,
              int64_t ng, int64_t mst, bool upper) {
  constexpr int NB = LdlBlock<T>::NB;
  // ng matrices mst elements apart (out and w alike) as blockIdx.z
  if (upper) {  // U = L^T (unit diagonal only)
    if (size != 1) return GPTQ2D_EUNSUPPORTED;
    const dim3 grid((unsigned)cdiv(k, 32), (unsigned)cdiv(k, 32), (unsigned)ng);
    hipLaunchKernelGGL(normalize_unit_upper_kernel<T>, grid, dim3(256), 0, stream, out, w, k, base, rs, cs, mst);
  } else if (size == 1) {
    const dim3 grid((unsigned)cdiv(k, 32), (unsigned)cdiv(k, 32), (unsigned)ng);
    hipLaunchKernelGGL(normalize_unit_kernel<T>, grid, dim3(256), 0, stream, out, w, k, base, rs, cs, mst);
  } else {
    constexpr int SB = LdlBlock<T>::SB;
    if (size > SB) return GPTQ2D_EUNSUPPORTED;
    const dim3 grid((unsigned)(k / size), (unsigned)cdiv(k, 64), (unsigned)ng);
    if (size <= NB)
      hipLaunchKernelGGL((normalize_block_kernel<T, NB>), grid, dim3(256), 0, stream, out, w, k, (int)size, base, rs,
                         cs, mst);
    else
      hipLaunchKernelGGL((normalize_block_solve_kernel<T, SB>), grid, dim3(256), 0, stream, out, w, k, (int)size,
                         base, rs, cs, mst);
  }
  return (int)hipGetLastError();
}

// One matrix of ldl_of_inverse in parts: col_begin == 0 starts it (the reversed copy into work);
// Cholesky panels [col_begin, col_end) (multiples of the panel width, col_end < 0 or >= k: to the
// end); finish: the triangular inverse and the normalisation into out (its three parts in order).
template <typename T>
int ldl_of_inverse_part(const T* m, T* out, T* work, int* info, int64_t k, int64_t size, int64_t col_begin,
                        int64_t col_end, bool finish, hipStream_t stream) {
  constexpr int PB = LdlBlock<T>::PB;
  if (k < 0 || size <= 0 || (k > 0 && k % size)) return GPTQ2D_EINVAL;
  if (size > 1 && size > LdlBlock<T>::SB) return GPTQ2D_EUNSUPPORTED;
  // range ends on panel boundaries, or at k (col_begin = k: nothing left to factor)
  if (col_begin < 0 || (col_begin % PB && col_begin != k) || (col_end >= 0 && col_end < col_begin) ||
      (col_end >= 0 && col_end % PB && col_end < k))
    return GPTQ2D_EINVAL;
  if (k == 0) {
    if (col_begin == 0) hipLaunchKernelGGL(zero_info_kernel, dim3(1), dim3(64), 0, stream, info, (int64_t)1);
    return (int)hipGetLastError();
  }
  int rc;
  const int64_t kk = k * k;
  if (col_begin == 0) {
    const int64_t blocks = cdiv(kk, 256) < 8192 ? cdiv(kk, 256) : 8192;
    hipLaunchKernelGGL(copy_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, work, m, kk, 1, info, 1);
    if ((rc = (int)hipGetLastError())) return rc;
  }
  if (col_begin < k &&
      (rc = cholesky_inplace<T>(work, k, info, out + stage_offset<T>(k), stream, col_begin, col_end)))
    return rc;
  if (finish)
    for (int phase = 1; phase <= 3; ++phase)
      if ((rc = trtri_part<T>(out, work, k, size, phase, stream))) return rc;
  return 0;
}

// Four events of the current device for this host thread (no timing), created on first use and
// kept until the process ends.
int pair_events(hipEvent_t (&ev)[4]) {
  thread_local std::unordered_map<int, std::array<hipEvent_t, 4>> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return GPTQ2D_EUNSUPPORTED;
  auto it = cache.find(dev);
  if (it == cache.end()) {
    std::array<hipEvent_t, 4> e{};
    for (auto& x : e)
      if (hipEventCreateWithFlags(&x, hipEventDisableTiming) != hipSuccess) return GPTQ2D_EUNSUPPORTED;
    it = cache.emplace(dev, e).first;
  }
  for (int i = 0; i < 4; ++i) ev[i] = it->second[i];
  return 0;
}

// ldl_of_inverse of two matrices at once (m[f], k[f] x k[f], block size size[f]; outputs out[f],
// scratch work[f], info[f]), on the caller's streams: factor f on stream[f], the first parts of the
// triangular inverses on stream[2].  One host loop enqueues the two Cholesky factorisations panel by
// panel, alternating, so that both chains of latency-bound panel launches are in flight together
// from the start; when a factorisation has passed its inverse's split point, part 1 of that inverse
// goes to stream[2] (after an event on stream[f]), where it runs beside the rest of both
// factorisations; parts 2 and 3 follow on stream[f], part 3 after an event on stream[2].  Two fp32
// matrices of one size on the two-level path share every Cholesky launch instead (CholeskyRun's
// twin).  The results equal two ldl_of_inverse calls bit for bit (each matrix sees the same
// workgroups' arithmetic, in another order of launches).
template <typename T>
int ldl_of_inverse_pair(const T* const* m, T* const* out, T* const* work, int* const* info, const int64_t* k,
                        const int64_t* size, bool upper1, hipStream_t const* stream) {
  for (int f = 0; f < 2; ++f) {
    if (k[f] < 0 || size[f] <= 0 || (k[f] > 0 && k[f] % size[f])) return GPTQ2D_EINVAL;
    if (size[f] > 1 && size[f] > LdlBlock<T>::NB) return GPTQ2D_EUNSUPPORTED;
  }
  if (upper1 && size[1] != 1) return GPTQ2D_EUNSUPPORTED;  // U = L^T: unit diagonal only
  if (stream[0] == stream[1] || stream[0] == stream[2] || stream[1] == stream[2]) return GPTQ2D_EINVAL;
  hipEvent_t ev[4];  // per factor: Cholesky past the split (on stream[f]), part 1 done (on stream[2])
  int rc;
  if ((rc = pair_events(ev))) return rc;
  int64_t split[2];
  CholeskyRun<T> twin(work[0], k[0], info[0], out[0] + stage_offset<T>(k[0]), stream[0]);
  const bool twinned = k[0] == k[1] && k[0] > 0 && twin.twin(work[1], info[1], out[1] + stage_offset<T>(k[1]));
  for (int f = 0; f < 2; ++f) {
    split[f] = k[f] > 0 ? trtri_split<T>(k[f]) : 0;
    if (k[f] == 0) {
      hipLaunchKernelGGL(zero_info_kernel, dim3(1), dim3(64), 0, stream[f], info[f], (int64_t)1);
      if ((rc = (int)hipGetLastError())) return rc;
      continue;
    }
    const int64_t kk = k[f] * k[f];
    const int64_t blocks = cdiv(kk, 256) < 8192 ? cdiv(kk, 256) : 8192;
    hipLaunchKernelGGL(copy_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream[twinned ? 0 : f], work[f], m[f],
                       kk, 1, info[f], 1);
    if ((rc = (int)hipGetLastError())) return rc;
  }
  if (twinned) {
    // both factorisations in one chain of launches on stream[0]; past the split, part 1 of the
    // inverses on stream[2] (factor 0) and stream[1] (factor 1), beside the rest of the chain; parts 2
    // and 3 of factor f on stream[f] after the chain (an event for stream[1]), part 3 of factor 0
    // after its part 1 (an event on stream[2])
    bool lead = split[0] == 0;
    while (!twin.done || !lead) {
      if ((rc = twin.step())) return rc;
      if (!lead && (twin.done || twin.j0 >= split[0])) {
        if ((rc = twin.flush_staged())) return rc;
        if (hipEventRecord(ev[0], stream[0]) != hipSuccess || hipStreamWaitEvent(stream[2], ev[0], 0) != hipSuccess ||
            hipStreamWaitEvent(stream[1], ev[0], 0) != hipSuccess)
          return GPTQ2D_EUNSUPPORTED;
        if ((rc = trtri_part<T>(out[0], work[0], k[0], size[0], 1, stream[2]))) return rc;
        if (hipEventRecord(ev[2], stream[2]) != hipSuccess) return GPTQ2D_EUNSUPPORTED;
        if ((rc = trtri_part<T>(out[1], work[1], k[1], size[1], 1, stream[1]))) return rc;
        lead = true;
      }
    }
    if (hipEventRecord(ev[1], stream[0]) != hipSuccess || hipStreamWaitEvent(stream[1], ev[1], 0) != hipSuccess)
      return GPTQ2D_EUNSUPPORTED;
    for (int f = 0; f < 2; ++f) {
      if ((rc = trtri_part<T>(out[f], work[f], k[f], size[f], 2, stream[f]))) return rc;
      if (f == 0 && split[0] && hipStreamWaitEvent(stream[0], ev[2], 0) != hipSuccess) return GPTQ2D_EUNSUPPORTED;
      if ((rc = trtri_part<T>(out[f], work[f], k[f], size[f], 3, stream[f], 1, f == 1 && upper1))) return rc;
    }
    return 0;
  }
  CholeskyRun<T> run[2] = {
      CholeskyRun<T>(work[0], k[0], info[0], out[0] + stage_offset<T>(k[0]), stream[0]),
      CholeskyRun<T>(work[1], k[1], info[1], out[1] + stage_offset<T>(k[1]), stream[1])};
  bool lead[2] = {split[0] == 0, split[1] == 0};  // part 1 enqueued (or none)
  while (!run[0].done || !run[1].done || !lead[0] || !lead[1]) {
    for (int f = 0; f < 2; ++f) {
      if ((rc = run[f].step())) return rc;
      // columns < split final: every panel before the split factored and its block copied into W
      // (fp32: the strip launch of the panel before the split does the copy; fp64: flush_staged)
      if (!lead[f] && (run[f].done || run[f].j0 >= split[f])) {
        if ((rc = run[f].flush_staged())) return rc;
        if (hipEventRecord(ev[f], stream[f]) != hipSuccess || hipStreamWaitEvent(stream[2], ev[f], 0) != hipSuccess)
          return GPTQ2D_EUNSUPPORTED;
        if ((rc = trtri_part<T>(out[f], work[f], k[f], size[f], 1, stream[2]))) return rc;
        if (hipEventRecord(ev[2 + f], stream[2]) != hipSuccess) return GPTQ2D_EUNSUPPORTED;
        lead[f] = true;
      }
    }
  }
  for (int f = 0; f < 2; ++f) {
    if (k[f] == 0) continue;
    if ((rc = trtri_part<T>(out[f], work[f], k[f], size[f], 2, stream[f]))) return rc;
    if (split[f] && hipStreamWaitEvent(stream[f], ev[2 + f], 0) != hipSuccess) return GPTQ2D_EUNSUPPORTED;
    if ((rc = trtri_part<T>(out[f], work[f], k[f], size[f], 3, stream[f], 1, f == 1 && upper1))) return rc;
  }
  return 0;
}

// inverse != 0: ldl_of_inverse; else ldl.  m, out, work: [batch, k, k] contiguous; info: [batch].
template <typename T>
int ldl_impl(bool inverse, const T* m, T* out, T* work, int* info, int64_t batch, int64_t k, int64_t size,
             hipStream_t stream) {
  if (batch < 0 || k < 0 || size <= 0 || (k > 0 && k % size)) return GPTQ2D_EINVAL;
  if (size > 1 && size > LdlBlock<T>::SB) return GPTQ2D_EUNSUPPORTED;
  if (batch == 0) return 0;
  if (k == 0) {
    hipLaunchKernelGGL(zero_info_kernel, dim3((unsigned)(cdiv(batch, 256) < 1024 ? cdiv(batch, 256) : 1024)), dim3(256),
                       0, stream, info, batch);
    return (int)hipGetLastError();
  }
  int rc;
  const int64_t kk = k * k;
  const int64_t blocks = cdiv(kk, 256) < 8192 ? cdiv(kk, 256) : 8192;
  // matrices taken in groups that share every Cholesky launch (CholeskyRun::twin; one at a time off the
  // fp32 two-level path): one chain of latency-bound panel launches per group instead of per matrix.
  // out[b] is free until the inverse / normalisation: its last elements stage the factored diagonal blocks.
  for (int64_t b0 = 0; b0 < batch;) {
    CholeskyRun<T> run(work + b0 * kk, k, info + b0, out + b0 * kk + stage_offset<T>(k), stream);
    int64_t nb = 1;
    while (b0 + nb < batch &&
           run.twin(work + (b0 + nb) * kk, info + b0 + nb, out + (b0 + nb) * kk + stage_offset<T>(k)))
      ++nb;
    for (int64_t b = b0; b < b0 + nb; ++b) {
      hipLaunchKernelGGL(copy_kernel<T>, dim3((unsigned)blocks), dim3(256), 0, stream, work + b * kk, m + b * kk, kk,
                         inverse ? 1 : 0, info + b, 1);
      if ((rc = (int)hipGetLastError())) return rc;
    }
    while (!run.done)
      if ((rc = run.step())) return rc;
    // the group's inverses and normalisations, each step one launch for the group
    if (inverse) {
      for (int phase = 1; phase <= 3; ++phase)
        if ((rc = trtri_part<T>(out + b0 * kk, work + b0 * kk, k, size, phase, stream, nb))) return rc;
    } else {
      if ((rc = normalize<T>(out + b0 * kk, work + b0 * kk, k, size, 0, k, 1, stream, nb, kk))) return rc;
    }
    b0 += nb;
  }
  return 0;
}

}  // namespace

extern "C" {

#define GPTQ2D_LDL_ABI(SUF, T)                                                                                      \
  int gptq2d_ldl_of_inverse_##SUF(const T* m, T* out, T* work, int* info, int64_t batch, int64_t k, int64_t size,  \
                                  hipStream_t stream) {                                                            \
    return ldl_impl<T>(true, m, out, work, info, batch, k, size, stream);                                            \
  }                                                                                                                 \
  int gptq2d_ldl_##SUF(const T* m, T* out, T* work, int* info, int64_t batch, int64_t k, int64_t size,              \
                       hipStream_t stream) {                                                                       \
    return ldl_impl<T>(false, m, out, work, info, batch, k, size, stream);                                           \
  }

GPTQ2D_LDL_ABI(f32, float)
GPTQ2D_LDL_ABI(f64, double)

#define GPTQ2D_LDL_PART_ABI(SUF, T)                                                                                 \
  int gptq2d_ldl_of_inverse_part_##SUF(const T* m, T* out, T* work, int* info, int64_t k, int64_t size,            \
                                       int64_t col_begin, int64_t col_end, int32_t finish, hipStream_t stream) {  \
    return ldl_of_inverse_part<T>(m, out, work, info, k, size, col_begin, col_end, finish != 0, stream);            \
  }                                                                                                                 \
  int gptq2d_ldl_of_inverse_pair_##SUF(const T* m0, T* out0, T* work0, int* info0, int64_t k0, int64_t size0,      \
                                       const T* m1, T* out1, T* work1, int* info1, int64_t k1, int64_t size1,      \
                                       int32_t upper1, hipStream_t stream0, hipStream_t stream1,                   \
                                       hipStream_t stream2) {                                                      \
    const T* m[2] = {m0, m1};                                                                                       \
    T* out[2] = {out0, out1};                                                                                       \
    T* work[2] = {work0, work1};                                                                                    \
    int* info[2] = {info0, info1};                                                                                  \
    const int64_t k[2] = {k0, k1}, size[2] = {size0, size1};                                                        \
    const hipStream_t st[3] = {stream0, stream1, stream2};                                                          \
    return ldl_of_inverse_pair<T>(m, out, work, info, k, size, upper1 != 0, st);                                     \
  }

GPTQ2D_LDL_PART_ABI(f32, float)
GPTQ2D_LDL_PART_ABI(f64, double)

}  // extern "C"
