// Fused GPTQ-2D sweep for per-entry quantizers (round, affine, teacher-forced codes).
//
// The matrix is cut into TR x TR tiles.  GPTQ-2D gives the same rounding for any order of the
// entries that respects the partial order (i' <= i, j' <= j), so the sweep runs over coarse
// stages T = I + J of tiles: the tiles of one coarse stage do not depend on each other, and each
// is swept by one workgroup entirely in LDS -- its 2*TR-1 antidiagonals one after another, every
// entry of an antidiagonal at once, the in-tile error feedback through the diagonal blocks
// L[I,I] and U[J,J], the quantizer applied in place.  Feedback between tiles: after each outer
// block of `outer_tiles` coarse stages, the block flush of flush.hip with P = Q = TR (on MFMA) into
// all later stages; inside an outer block, fp32 tiles pull the feedback of the block's earlier tiles
// on MFMA (tile_stage_kernel), fp64 stages are flushed into the rest of the block after each coarse
// stage (sweep_tile64_kernel then sweeps).  Both run the same push-form in-tile sweep (sweep_tile).
// The host loop below issues every launch of the sweep from C++ in one call, so a whole layer is one
// C-ABI call and one capturable stream of kernels.
//
// In exact arithmetic the result equals the reference's blocked sweep (gptq_2d.py:1295-1375) and
// Algorithm 1 on vec(X) (GPTQ-2D paper, Theorem 1); in floating point the sums are accumulated in
// a different order.  The in-tile value of entry (r, c) when it is rounded is
//   y = (Y[r,c] + sum_{r'<r} L[r,r'] E[r',c]) + sum_{c'<c} C[r,c'] U[c',c]
// where C[r,c'] is already complete (all rows above in the tile were rounded earlier).
#include "common.h"
#include "lds_dma.h"
#include "profile.h"

#include <mutex>
#include <type_traits>
#include <utility>

template <typename T>
int gptq2d_flush(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t P, int64_t Q,
                 int64_t s0, int64_t s1, int64_t s_end, const BatchMap& lmap, const BatchMap& umap, int64_t B,
                 hipStream_t stream);
template <typename T>
int gptq2d_fill(T* x, T v, int64_t count, hipStream_t stream);
int gptq2d_flush_kron(float* y, float* c, const float* e, const float* l, const KronU& kr, int64_t m, int64_t n,
                      int64_t s0, int64_t s1, int64_t s_end, hipStream_t stream);

namespace {

constexpr int TR = 32;       // tile edge
constexpr int64_t BAND64 = 4;  // fp64 fused sweep: tile stages per band flush inside an outer block
constexpr int PARTS = 8;     // threads cooperating on one entry of an antidiagonal
constexpr int NTHREADS = TR * PARTS;

// Q_ABSMAX: the abs-max INT quantizer of a super-entry row (int_abs_max_quantizer, quantizer_int.py:120-134),
// only with 1 x TR super-entries.
enum QKind : int32_t { Q_ROUND = 0, Q_AFFINE = 1, Q_FORCED = 2, Q_ABSMAX = 3 };

template <typename T>
struct QSpec {
  int32_t kind;
  const T* scale;  // affine: full [*, m, n] scale; forced: the codes' values
  const T* zp;     // affine: full [*, m, n] zero point
  BatchMap smap, zmap;
  T qmin, qmax;
  T* ypre;          // optional [B, m, n]: Y of every entry just before it is rounded
  T* sout;          // abs-max, optional [B, m, n]: the scale each entry's row was rounded with
  int32_t dtype16;  // abs-max: the scale's 16-bit type (1 bf16, 2 fp16)
};

// f(integral_constant<int, I>) for I = 0, 1, ..., in order: a loop whose index is a compile-time constant in
// every iteration.
template <typename F, int... I>
__device__ __forceinline__ void static_for(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}

// The affine quantizer (clamp(round(y / s + z), qmin, qmax) - z) s by IEEE division, the dequantized value
// rounded on its own (as the reference's plug-in writes it), so that a caller's error z - y is exactly that
// difference: no contraction of the product into the caller's subtraction.
template <typename T>
__device__ __forceinline__ T quantize_entry_div(T yv, T sv, T zv, T qmin, T qmax) {
#pragma clang fp contract(off)
  const T code = clamp_val(round_even(yv / sv + zv), qmin, qmax);
  return (code - zv) * sv;
}

// The abs-max quantizer clamp(round(y / s), qmin, qmax) s of quantizer_int.py:134 (the product is exact for
// a 16-bit scale and a small code, and rounded on its own in any case).
template <typename T>
__device__ __forceinline__ T quantize_absmax_entry(T yv, T sv, T qmin, T qmax) {
#pragma clang fp contract(off)
  return clamp_val(round_even(yv / sv), qmin, qmax) * sv;
}

// ------------------------------------------------------------------------------------------------ 1 x TR super-entries
//
// With super-entries of one row and TR columns (gptq_2d_super_entry with super_entry_shape (1, TR), e.g. the
// three-factor layer's 1 x 32 abs-max groups) a tile holds the TR super-entries (i0 + r, J) of one coarse
// column, ordered by row; the tiles' coarse stages and the feedback between tiles (pulls, flushes) are
// those of plain entries, and U's TR x TR diagonal blocks -- identity by the super-entry convention -- are
// never read.  Inside a tile the sweep is TR steps, one per row: the row's entries are rounded jointly
// from y = Y + down (the in-tile feedback through L[I,I]), then their errors are pushed to the rows below.
// Thread (g, c) = (tid / 32, tid % 32) owns column c of rows 4g .. 4g + 3; a row is the 32 lanes of one
// half-wave, so the abs-max of a super-entry row is a half-wave reduction.

// Maximum over the 32 lanes of each half-wave (all of them receive it).
template <typename T>
__device__ __forceinline__ T halfwave_max(T v) {
#pragma unroll
  for (int k = 16; k >= 1; k >>= 1) {
    const T o = __shfl_xor(v, k, 32);
    v = o > v ? o : v;
  }
  return v;
}

// The rows' quantizer inputs (affine: scale and zero point; forced: the values), read from global memory
// at the start of the kernel.
template <typename T, int KIND>
struct RowInputs {
  T s[4], z[4];

  __device__ __forceinline__ void load(const QSpec<T>& qs, int64_t b, int64_t m, int64_t n, int64_t i0, int64_t j0) {
    const int cc = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int rows_in = m - i0 < TR ? (int)(m - i0) : TR;
    const int64_t corner = i0 * n + j0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 4 * g + i;
      const bool in = r < rows_in;
      const int64_t off = corner + (int64_t)r * n + cc;
      s[i] = z[i] = T(0);
      if constexpr (KIND == Q_AFFINE) {
        s[i] = in ? qs.scale[qs.smap.offset(b) + off] : T(1);
        z[i] = in ? qs.zp[qs.zmap.offset(b) + off] : T(0);
      } else if constexpr (KIND == Q_FORCED) {
        s[i] = in ? qs.scale[qs.smap.offset(b) + off] : T(0);
      }
    }
  }
};

// The TR row steps of one tile, then its Y, C and E to global memory.  ys / cs: the tile's Y and C with
// the pulled feedback (row pitches ysp, csp); lp[r lpp + k] = L[i0 + r, i0 + k] for k < r, zero
// elsewhere; es: TR x esp floats for the published errors.  Expects the image complete (a barrier after
// it was written).
template <typename T, int KIND, bool YPRE>
__device__ __forceinline__ void sweep_rows(const T* ys, int ysp, const T* cs, int csp, const T* lp, int lpp, T* es,
                                           int esp, const RowInputs<T, KIND>& in, T* __restrict__ y,
                                           T* __restrict__ c, T* __restrict__ e, const QSpec<T>& qs, int64_t m,
                                           int64_t n, int64_t i0, int64_t j0, int64_t mat) {
  const int cc = threadIdx.x & 31, g = threadIdx.x >> 5;
  const int rows_in = m - i0 < TR ? (int)(m - i0) : TR;  // the super-entries span the tile's columns
  T Y[4], C[4], D[4], E[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    Y[i] = ys[(4 * g + i) * ysp + cc];
    C[i] = cs[(4 * g + i) * csp + cc];
    D[i] = E[i] = T(0);
  }
  const T qmin = qs.qmin, qmax = qs.qmax, half = (qs.qmax - qs.qmin) / T(2);
  auto step = [&](auto r_c) __attribute__((always_inline)) {
    constexpr int r = decltype(r_c)::value, slot = r & 3;
    const bool own = g == (r >> 2) && r < rows_in;
    const T yv = Y[slot] + D[slot];
    T z, sc = T(1);
    if constexpr (KIND == Q_ABSMAX) {
      // scale from the row's current abs max (a NaN entry counts as 0, as in the plug-in's comparison
      // loop), rounded to the 16-bit type through fp32, 0 -> 1; the reduction runs on every lane
      const T a = own ? __builtin_fmax(__builtin_fabs(yv), T(0)) : T(0);
      const T amax = halfwave_max(a);
      sc = round_scale16(amax / half, qs.dtype16);
      sc = sc == T(0) ? T(1) : sc;
      z = quantize_absmax_entry(yv, sc, qmin, qmax);
    } else if constexpr (KIND == Q_AFFINE) {
      // the dequantized value rounded on its own, before the error z - y (no contraction into it)
      z = quantize_entry_div(yv, in.s[slot], in.z[slot], qmin, qmax);
    } else if constexpr (KIND == Q_FORCED) {
      z = in.s[slot];
    } else {
      z = round_even(yv);
    }
    const T ev = z - yv;
    const T cf = (C[slot] + D[slot]) + ev;
    if (own) {
      Y[slot] = z;
      E[slot] = ev;
      C[slot] = cf;
      es[r * esp + cc] = ev;
      if constexpr (YPRE) qs.ypre[mat + (i0 + r) * n + j0 + cc] = yv;
      if constexpr (KIND == Q_ABSMAX) {
        if (qs.sout) qs.sout[mat + (i0 + r) * n + j0 + cc] = sc;
      }
    }
    if constexpr (r + 1 < TR) {
      __syncthreads();  // the row's errors before the rows below read them
      const T er = es[r * esp + cc];
#pragma unroll
      for (int i = 0; i < 4; ++i) D[i] += lp[(4 * g + i) * lpp + r] * er;
    }
  };
  static_for(step, std::make_integer_sequence<int, TR>{});
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 4 * g + i;
    if (r < rows_in) {
      const int64_t off = mat + (i0 + r) * n + j0 + cc;
      y[off] = Y[i];
      c[off] = C[i];
      e[off] = E[i];
    }
  }
}

// One launch per coarse stage of the row-super-entry sweep on the generic (fp64) path: each workgroup
// loads its tile's Y, C and L[I,I] and sweeps it (the feedback of earlier tiles was flushed in).
template <typename T, int KIND, bool YPRE>
__global__ __launch_bounds__(NTHREADS) void sweep_rows_kernel(T* __restrict__ y, T* __restrict__ c,
                                                              T* __restrict__ e, const T* __restrict__ l, int64_t m,
                                                              int64_t n, int64_t stage, int64_t tile_lo,
                                                              BatchMap lmap, QSpec<T> qs, int64_t nx, int64_t ny) {
  __shared__ T Ys[TR][TR + 1];
  __shared__ T Cs[TR][TR + 1];
  __shared__ T Ls[TR][TR + 1];
  __shared__ T Es[TR][TR + 1];
  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t I = tile_lo + id.x, J = stage - I;
  const int64_t i0 = I * TR, j0 = J * TR;
  const int64_t mat = b * m * n;
  const T* lb = l + lmap.offset(b);
  const int rows_in = m - i0 < TR ? (int)(m - i0) : TR;
  RowInputs<T, KIND> in;
  in.load(qs, b, m, n, i0, j0);
  for (int t = threadIdx.x; t < TR * TR; t += NTHREADS) {
    const int r = t / TR, cc = t % TR;
    const bool rin = r < rows_in;
    const int64_t off = mat + (i0 + r) * n + j0 + cc;
    Ys[r][cc] = rin ? y[off] : T(0);
    Cs[r][cc] = rin ? c[off] : T(0);
    Ls[r][cc] = (cc < r && rin) ? lb[(i0 + r) * m + i0 + cc] : T(0);  // strictly below the diagonal
  }
  __syncthreads();
  sweep_rows<T, KIND, YPRE>(&Ys[0][0], TR + 1, &Cs[0][0], TR + 1, &Ls[0][0], TR + 1, &Es[0][0], TR + 1, in, y, c, e, qs,
                            m, n, i0, j0, mat);
}


// ------------------------------------------------------------------------------------------------ fp32: pull + sweep

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Quantizer of the fused sweeps, applied to one value.
template <int KIND>
__device__ __forceinline__ float quantize_entry(float yv, float sv, float zv, float qmin, float qmax) {
  if constexpr (KIND == Q_AFFINE) {
    const float code = clamp_val(round_even(yv / sv + zv), qmin, qmax);
    return (code - zv) * sv;
  } else if constexpr (KIND == Q_FORCED) {
    return sv;
  } else {
    return round_even(yv);
  }
}

// One wave's share of a band product on MFMA: acc += sum over the k-chunks ch in [c_lo, c_hi) with
// ch = c_lo + part (mod nparts) of A[i0 + 0..31, 8 ch + 0..7] B[8 ch + 0..7, j0 + 0..31], A and B
// row-major (lda, ldb), read straight from global memory into the MFMA operand layout: lane l
// supplies A(l % 32, 8 ch + 4 (l / 32) + s) and B(8 ch + 4 (l / 32) + s, l % 32) to MFMA s = 0..3 of
// the chunk.  Loads of G chunks are issued before their MFMAs.
template <bool VEC>
__device__ __forceinline__ void pull_chunks(floatx16& acc, const float* __restrict__ A, int64_t lda, int64_t a_rows,
                                            int64_t a_cols, const float* __restrict__ Bm, int64_t ldb,
                                            int64_t b_rows, int64_t b_cols, int64_t i0, int64_t j0, int64_t c_lo,
                                            int64_t c_hi, int part, int nparts, int li, int hh) {
  // this lane's row of A and column of B as pointers (64-bit arithmetic once); k offsets in 32 bits
  const int64_t ia = i0 + li, jb = j0 + li;
  const bool arow = ia < a_rows, bcol = jb < b_cols;
  const float* ap = A + (arow ? ia : 0) * lda;
  const float* bp = Bm + (bcol ? jb : 0);
  const int clo = (int)c_lo, chi = (int)c_hi, acols = (int)a_cols, brows = (int)b_rows;
  constexpr int G = 4;
  for (int base = clo + part; base < chi; base += nparts * G) {
    float av[G][4], bv[G][4];
#pragma unroll
    for (int q = 0; q < G; ++q) {
      const int ch = base + nparts * q;
      const int k0 = 8 * ch + 4 * hh;
      const bool ok = ch < chi;
      if (VEC) {
        const float4 f = (ok && arow && k0 < acols) ? *reinterpret_cast<const float4*>(ap + k0)
                                                    : make_float4(0.f, 0.f, 0.f, 0.f);
        av[q][0] = f.x, av[q][1] = f.y, av[q][2] = f.z, av[q][3] = f.w;
      } else {
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) av[q][s2] = (ok && arow && k0 + s2 < acols) ? ap[k0 + s2] : 0.f;
      }
      const float* bk = bp + (int64_t)k0 * ldb;
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) bv[q][s2] = (ok && bcol && k0 + s2 < brows) ? bk[s2 * ldb] : 0.f;
    }
#pragma unroll
    for (int q = 0; q < G; ++q) {
      if (base + nparts * q >= chi) break;
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][s2], bv[q][s2], acc, 0, 0, 0);
    }
  }
}

// pull_chunks for the right product R = C U with U = P (x) Q given by its factors (nq % 16 == 0): B value (k, j)
// is Q[k % nq, j % nq] times P[k / nq, j / nq] -- one fp32 multiplication, the entry of the explicit product bit
// for bit.  A lane's column is fixed, and an 8-row chunk lies in one block of P, so each chunk takes one P entry
// per lane; the chunk's 16-row unit is split on the scalar unit.  Q is read through a buffer resource based at
// the chunk's first row (the lane's column in the vector offset, the row step in the scalar one, a lane past
// the matrix masked by an offset beyond the extent): no branches and no 64-bit address arithmetic per load.
// Every row a chunk reads lies below n (the right product's k-tiles are t < J <= nt - 1).
template <bool VEC>
__device__ __forceinline__ void pull_chunks_kron(floatx16& acc, const float* __restrict__ A, int64_t lda,
                                                 int64_t a_rows, int64_t a_cols, const KronU& kr, int64_t b_rows,
                                                 int64_t b_cols, int64_t i0, int64_t j0, int64_t c_lo, int64_t c_hi,
                                                 int part, int nparts, int li, int hh) {
  const int64_t ia = i0 + li, jb = j0 + li;
  const bool arow = ia < a_rows, bcol = jb < b_cols;
  const float* ap = A + (arow ? ia : 0) * lda;
  int pj = 0, qj = 0;  // the lane's column: block of P, column of Q
  if (bcol) kron_index(kr, (int)jb, pj, qj);
  // the tile's columns in one block of P (all but the tiles that straddle a block edge): the chunks' P entries
  // are read through the scalar cache
  int pu0, pu1, qu;
  kron_index(kr, (int)j0, pu0, qu);
  kron_index(kr, (int)(j0 + TR - 1 < b_cols - 1 ? j0 + TR - 1 : b_cols - 1), pu1, qu);
  const int nq = kr.nq;
  const int qoff = bcol ? (qj + 4 * hh * nq) * 4 : OOB;  // bytes: the lane's column of Q, its k slot
  const float* pp = kr.p + pj;
  const int clo = (int)c_lo, chi = (int)c_hi, acols = (int)a_cols;
  const int upart = __builtin_amdgcn_readfirstlane(part), unparts = __builtin_amdgcn_readfirstlane(nparts);
  constexpr int G = 4;
  auto run = [&](auto uniform_c) {
    constexpr bool UNI = decltype(uniform_c)::value;
    for (int base = clo + upart; base < chi; base += unparts * G) {
      float av[G][4], bv[G][4], pv[G];
#pragma unroll
      for (int q = 0; q < G; ++q) {
        const int ch = base + unparts * q;
        const int k0 = 8 * ch + 4 * hh;
        const bool ok = ch < chi;
        if (VEC) {
          const float4 f = (ok && arow && k0 < acols) ? *reinterpret_cast<const float4*>(ap + k0)
                                                      : make_float4(0.f, 0.f, 0.f, 0.f);
          av[q][0] = f.x, av[q][1] = f.y, av[q][2] = f.z, av[q][3] = f.w;
        } else {
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) av[q][s2] = (ok && arow && k0 + s2 < acols) ? ap[k0 + s2] : 0.f;
        }
        int ub, ur;  // the chunk's rows: 16-row unit ch / 2 = block ub of P, rows 16 ur + 8 (ch % 2) + .. of Q
        kron_split(kr, (unsigned)(ok ? ch >> 1 : 0), ub, ur);
        if constexpr (UNI)
          pv[q] = kron_p_uniform(kr, ub * kr.np + pu0);
        else
          pv[q] = pp[ub * kr.np];
        const int row0 = 16 * ur + 8 * (ch & 1);
        const int64_t ext = ok ? (int64_t)(nq - row0) * nq : 0;  // elements from the chunk's first row
        const __amdgpu_buffer_rsrc_t qr =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(kr.q + (int64_t)row0 * nq), (short)0,
                                              (int)(ext < OOB / 4 ? ext * 4 : OOB), 0x00020000);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
          bv[q][s2] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(qr, qoff, s2 * nq * 4, 0));
      }
      // the products after all loads: a product inside a mask's branch would make each load wait for its data
      // before the next one issues
#pragma unroll
      for (int q = 0; q < G; ++q)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) bv[q][s2] *= pv[q];
#pragma unroll
      for (int q = 0; q < G; ++q) {
        if (base + unparts * q >= chi) break;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
          acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][s2], bv[q][s2], acc, 0, 0, 0);
      }
    }
  };
  if (pu0 == pu1)
    run(std::true_type{});
  else
    run(std::false_type{});
}

// LDS row pitch of the tile's Y and E images: 40 = 8 (mod 32) keeps the column walks of the E reads
// (a row step of 39 = -7 mod 32 banks between neighbouring columns) and the final row-wise stores free
// of bank conflicts beyond 2-way.
constexpr int SP = 40;

// LDS image of one tile for the fp32 in-tile sweep.  L[I,I] and U[J,J] are stored with zero padding so
// that the sweep reads them at any offset in [-TR, 2 TR) without masks:
// Lp[r][TR + k] = L[i0+r, i0+k] for 0 <= k < r (zero elsewhere), Up[TR + k][c] = U[j0+k, j0+c] for
// k < c (zero elsewhere).  Ys: the tile's Y with the pulled feedback (on entry), the result (at the end).
// Cs[r][TR + c] and Es[TR + r][c]: the C and E images, padded by TR zero columns (C) and rows (E) on
// each side: C holds C + pulled D on entry and each entry's final C from its rounding on; E holds
// zeros on entry and each entry's error from its rounding on.  The sweep reads both at offsets that
// leave the tile (times zero coefficients), so the padding must hold finite values.
// Row pitches of the padded L, U and C images: with 103, 39 and 98 floats every per-step read of the
// sweep (L[r, t - c], U[t - r, c], C[r, t - r] over a half-wave's 4 rows x 8 parts) falls on 32 distinct
// banks; the natural pitches (97, 33, 97) put 4 rows on one bank in each of them.
constexpr int LPW = 3 * TR + 7;
constexpr int UPW = TR + 7;
constexpr int CPW = 3 * TR + 2;
constexpr int EROWS = 3 * TR;

// (T = double: the same image in fp64; every pitch gives the 32 lanes of a half-wave 32 distinct positions
// mod 32, so their 64-bit reads cover the 64 banks once)
template <typename T>
struct TileLdsT {
  T Ys[TR][SP];  // first: the sweep's base pointers below reach up to 23 rows / columns before Lp and Up
  T Lp[TR][LPW];
  T Up[3 * TR][UPW];
  T Cs[TR][CPW];
  T Es[EROWS][SP];
};
using TileLds = TileLdsT<float>;

// Affine / round / forced quantizer of the in-tile sweep, given the precomputed correctly rounded
// reciprocal rv = 1/sv and whether sv lies in [2^-60, 2^60] (affine only).  y / s is formed as
// q0 = y rv, then one FMA correction with the exact remainder y - q0 s (Markstein's method): the
// IEEE quotient whenever also 2^-60 <= |y| < 2^61 (then no product or remainder over- or
// underflows: |q0| lies in [2^-121, 2^121] and the remainder is a multiple of 2^-107).  `exact` says
// whether that holds -- the biased exponent of y in [67, 187], one bit-field test (zero, denormal,
// infinite and NaN y fail it) -- and otherwise quantize_entry_div (the division itself) gives the
// value.  This keeps the division's ten dependent operations off the per-antidiagonal critical path.
//
__device__ __forceinline__ float fma_of(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_of(double a, double b, double c) { return __builtin_fma(a, b, c); }

// fp64: the same with 2^-500 <= |s| <= 2^500 and 2^-500 <= |y| < 2^501 (biased exponent of y in [523, 1523]):
// |q0| lies in [2^-1001, 2^1001] and the remainder is a multiple of 2^-605, all normal.
template <int KIND, typename T>
__device__ __forceinline__ T quantize_entry_rcp(T yv, T sv, T zv, T rv, bool s_ok, T qmin, T qmax, bool& exact) {
  // the dequantized value is rounded on its own (as the reference's plug-in writes it), so that the
  // caller's error z - y is exactly that difference: no contraction into the caller's subtraction
#pragma clang fp contract(off)
  if constexpr (KIND == Q_AFFINE) {
    const T q0 = yv * rv;
    const T rem = fma_of(-q0, sv, yv);
    const T q = fma_of(rem, rv, q0);
    // s_ok also holds only when the zero point is not NaN and qmin <= qmax: then q is the IEEE
    // quotient, round(q + z) is not NaN, and the median of (x, qmin, qmax) is the clamp, in one
    // operation on the per-step critical path
    if constexpr (sizeof(T) == 4) {
      const unsigned ex = (__float_as_uint(yv) >> 23) & 0xffu;
      exact = s_ok && ex - 67u <= 120u;
      const T code = __builtin_amdgcn_fmed3f(round_even(q + zv), qmin, qmax);
      return (code - zv) * sv;
    } else {
      const unsigned ex = (unsigned)(__builtin_bit_cast(unsigned long long, yv) >> 52) & 0x7ffu;
      exact = s_ok && ex - 523u <= 1000u;
      const T code = clamp_val(round_even(q + zv), qmin, qmax);
      return (code - zv) * sv;
    }
  } else if constexpr (KIND == Q_FORCED) {
    exact = true;
    return sv;
  } else {
    exact = true;
    return round_even(yv);
  }
}


// Thread ownership of the in-tile sweep.  Thread (r, part) = (tid / 8, tid % 8) owns the four entries
// (r, c) of its row with (c + r) % 8 == part; slot j holds the one whose antidiagonal t_e = r + c has
// (t_e / 8) % 4 == j.  The entry rounded at step t is then slot (t / 8) % 4 of part t % 8 in every row: a
// compile-time register in the unrolled loop over t.
__device__ __forceinline__ void slot_columns(int r, int part, int (&cs)[4]) {
  const int qlo = (r - part + 7) >> 3;  // smallest q with 8 q + part >= r
#pragma unroll
  for (int j = 0; j < 4; ++j) cs[j] = 8 * (qlo + ((j - qlo) & 3)) + part - r;  // in [0, TR)
}

// Quantizer inputs of the sweep's entries in its own layout (slot order), read from global memory at
// the start of the kernel so that their latency overlaps the pull.
template <int KIND, typename T = float>
struct SweepInputs {
  T s[4], z[4];

  __device__ __forceinline__ void load(const QSpec<T>& qs, int64_t b, int64_t m, int64_t n, int64_t i0,
                                       int64_t j0) {
    const int tid = threadIdx.x, r = tid >> 3, part = tid & 7;
    int cs[4];
    slot_columns(r, part, cs);
    const int rows_in = m - i0 < TR ? (int)(m - i0) : TR, cols_in = n - j0 < TR ? (int)(n - j0) : TR;
    const int64_t corner = i0 * n + j0;
    const T* st = KIND != Q_ROUND ? qs.scale + qs.smap.offset(b) + corner : nullptr;
    const T* zt = KIND == Q_AFFINE ? qs.zp + qs.zmap.offset(b) + corner : nullptr;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool in = r < rows_in && cs[j] < cols_in;
      const int off = r * (int)n + cs[j];
      s[j] = z[j] = T(0);
      if constexpr (KIND == Q_AFFINE) {
        s[j] = in ? st[off] : T(1);
        z[j] = in ? zt[off] : T(0);
      } else if constexpr (KIND == Q_FORCED) {
        s[j] = in ? st[off] : T(0);
      }
    }
  }
};

// The tile's 63 antidiagonals, in push form.  A step: the rounding lanes quantize (their entries'
// feedback is complete) and write the error into the E image and the final C into the C image; one
// workgroup barrier; then every lane reads the step's error in each of its columns (E[t - c, c]) and
// the final C of its row (C[r, t - r]) and adds the step's feedback to its entries' sums -- down:
// L[r, t-c] E[t-c, c], right: C[r, t-r] U[t-r, c].  An entry is rounded at y = (Y + down) + right,
// and its C becomes (C + down) + error.  The zero-padded diagonal blocks make the terms vanish for
// entries already rounded, for sources below the entry (not yet written in the images: their zeros or
// values times zero) and for sources outside the tile.  Then Y, C and E of the tile go to global
// memory.  Expects the tile image complete in LDS (a barrier after it was written).
//
// The step is bound by its chain (the quantizer's ~13 dependent operations, the LDS write, barrier
// and read-back, ~150 clocks measured for the exchange alone) and by the LDS reads of four waves
// (13 per lane); the image pitches keep every read free of bank conflicts.
template <int KIND, bool YPRE, typename T>
__device__ __forceinline__ void sweep_tile(TileLdsT<T>& tl, const SweepInputs<KIND, T>& in, T* __restrict__ y,
                                           T* __restrict__ c, T* __restrict__ e, const QSpec<T>& qs, int64_t m,
                                           int64_t n, int64_t i0, int64_t j0, int64_t mat) {
  const int tid = threadIdx.x;
  const int r = tid >> 3, part = tid & 7;
  const int rows_in = m - i0 < TR ? (int)(m - i0) : TR;  // tile rows / columns inside the matrix
  const int cols_in = n - j0 < TR ? (int)(n - j0) : TR;
  const bool row_in = r < rows_in;
  int cs[4];
  slot_columns(r, part, cs);
  // per entry: Y and C on entry, the in-tile down and right feedback sums D and F (kept apart from
  // Y, so that their rounding errors scale with the feedback, not with Y), the error E, the
  // quantizer inputs S, Z and the reciprocal R of S, and the step at which the entry is rounded (-1
  // for entries outside the matrix)
  T Y[4], C[4], D[4], F[4], E[4], S[4], Z[4], R[4];
  int tr[4];
  bool s_ok[4];
  const bool qmin_le_qmax = qs.qmin <= qs.qmax;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    tr[j] = row_in && cs[j] < cols_in ? r + cs[j] : -1;
    Y[j] = tl.Ys[r][cs[j]];
    C[j] = tl.Cs[r][TR + cs[j]];
    D[j] = F[j] = E[j] = T(0);
    S[j] = in.s[j];
    Z[j] = in.z[j];
    R[j] = T(0);
    s_ok[j] = false;
    if constexpr (KIND == Q_AFFINE) {
      R[j] = T(1) / S[j];
      T as;
      if constexpr (sizeof(T) == 4)
        as = __builtin_fabsf(S[j]);
      else
        as = __builtin_fabs(S[j]);
      // the range in which the quotient from the reciprocal is the IEEE one (quantize_entry_rcp)
      constexpr T s_lo = sizeof(T) == 4 ? T(0x1p-60) : T(0x1p-500), s_hi = sizeof(T) == 4 ? T(0x1p60) : T(0x1p500);
      s_ok[j] = as >= s_lo && as <= s_hi && Z[j] == Z[j] && qmin_le_qmax;
    }
  }
  T* ypre_row = YPRE ? qs.ypre + mat + (i0 + r) * n + j0 : nullptr;
  // clamp bounds pinned in registers (an empty asm makes them opaque): otherwise the compiler
  // re-reads them from the kernel arguments on every step
  T qmin = qs.qmin, qmax = qs.qmax;
  asm volatile("" : "+v"(qmin), "+v"(qmax));
  // what a thread reads and writes at step t, as pointers plus t or t times the row pitch (immediate
  // offsets): the C of its row's rounded entry C[r, t - r] (which the rounding lane writes), that
  // lane's E[r, t - r], and per slot the source E[t - c, c] and the coefficients L[r, t - c], U[t - r, c]
  T* const cp = &tl.Cs[r][TR] - r;
  T* const ewp = &tl.Es[TR + r][0] - r;
  const T* ep[4];
  const T* lp[4];
  const T* up[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    ep[j] = &tl.Es[TR][0] + (cs[j] - cs[j] * SP);
    lp[j] = &tl.Lp[r][TR] - cs[j];
    up[j] = &tl.Up[TR][0] + (cs[j] - r * UPW);
  }
  constexpr int STEPS = 2 * TR - 1;
  // L and U coefficients of step t in LV[t & 1], UV[t & 1], read a step ahead (they do not depend on
  // the sweep), so that only the published errors and C are read between the barrier and the
  // feedback update, and no register copies are needed in the unrolled loop
  T LV[2][4], UV[2][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    LV[0][j] = lp[j][0];
    UV[0][j] = up[j][0];
  }
  // one step at compile-time index t (the loop is unrolled by a fold over the steps: the register slot,
  // the parity buffers and the LDS immediates are compile-time in every step)
  auto step = [&](auto t_c) __attribute__((always_inline)) {
    constexpr int t = decltype(t_c)::value;
    constexpr int cur = t & 1, ka = (t >> 3) & 3;
    // every lane evaluates its step's register; only the rounding lanes keep and publish it
    const bool rnd = tr[ka] == t;
    const T yv = (Y[ka] + D[ka]) + F[ka];
    {
      bool exact;
      T z = quantize_entry_rcp<KIND>(yv, S[ka], Z[ka], R[ka], s_ok[ka], qmin, qmax, exact);
      T ev = z - yv;
      const T cd = C[ka] + D[ka];
      T cf = cd + ev;
      if (rnd) {
        // published at once; a lane whose quotient needs the division writes again (same address:
        // the later write stands), behind a branch taken only when some lane of the wave needs it
        ewp[t] = ev;
        cp[t] = cf;
        if constexpr (KIND == Q_AFFINE) {
          if (__builtin_amdgcn_ballot_w64(!exact)) {
            asm volatile("");  // keeps the division behind the branch (no speculation into a select)
            if (!exact) {
              z = quantize_entry_div(yv, S[ka], Z[ka], qmin, qmax);
              ev = z - yv;
              cf = cd + ev;
              ewp[t] = ev;
              cp[t] = cf;
            }
          }
        }
        Y[ka] = z;
        E[ka] = ev;
        C[ka] = cf;
      }
    }
    if constexpr (t == STEPS - 1) {
      if constexpr (YPRE) {
        if (rnd) ypre_row[t - r] = yv;
      }
      return;  // nothing left to receive feedback
    }
    __syncthreads();  // every wave's writes of this step before any wave's reads
    const T cr = cp[t];
    T ev[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ev[j] = ep[j][t * SP];
    if constexpr (t + 1 < STEPS - 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        LV[cur ^ 1][j] = lp[j][t + 1];
        UV[cur ^ 1][j] = up[j][(t + 1) * UPW];
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      D[j] += LV[cur][j] * ev[j];
      F[j] += cr * UV[cur][j];
    }
    // the pre-quantization value out after the step's feedback is issued
    if constexpr (YPRE) {
      if (rnd) ypre_row[t - r] = yv;
    }
    // no second barrier: every image entry is written once (at its entry's step), so the next step's
    // writes never touch what this step reads
  };
  static_for(step, std::make_integer_sequence<int, STEPS>{});

#pragma unroll
  for (int j = 0; j < 4; ++j) tl.Ys[r][cs[j]] = Y[j];
  __syncthreads();
  T* yt = y + mat + i0 * n + j0;
  T* ct = c + mat + i0 * n + j0;
  T* et = e + mat + i0 * n + j0;
  for (int t = tid; t < TR * TR; t += NTHREADS) {
    const int rr = t / TR, cc = t % TR;
    if (rr < rows_in && cc < cols_in) {
      const int off = rr * (int)n + cc;
      yt[off] = tl.Ys[rr][cc];
      ct[off] = tl.Cs[rr][TR + cc];
      et[off] = tl.Es[TR + rr][cc];
    }
  }
}

// The pulled feedback at (r, cc) from the four waves' partial sums (wave w's in red[w / 2][w % 2]):
// waves [0, wd) summed the down product D, the others the right product R (in wave order).
__device__ __forceinline__ void pulled_sums(const float (*red)[2][TR][TR + 1], int wd, int r, int cc, float& dd,
                                            float& rr) {
  const float s0 = red[0][0][r][cc], s1 = red[0][1][r][cc], s2 = red[1][0][r][cc], s3 = red[1][1][r][cc];
  dd = (wd > 0 ? s0 : 0.f) + (wd > 1 ? s1 : 0.f) + (wd > 2 ? s2 : 0.f) + (wd > 3 ? s3 : 0.f);
  rr = (wd > 0 ? 0.f : s0) + (wd > 1 ? 0.f : s1) + (wd > 2 ? 0.f : s2) + (wd > 3 ? 0.f : s3);
}

// Own tile data of the fp32 kernels, read before the tile's feedback is complete (it does not
// depend on it): entry q of this thread is (t / TR, t % TR) with t = threadIdx.x + NTHREADS q.
// ROWS: the tile image of the row-super-entry sweep (1 x TR super-entries): no U block (identity by the
// super-entry convention, never read), no padding and no E image.
template <bool ROWS, typename T = float>
struct TileRegs {
  static constexpr int NQ = TR * TR / NTHREADS;
  T y[NQ], c[NQ], l[NQ], u[NQ];

  // KR (fp32): U given by its Kronecker factors (ub unused), each entry of the diagonal tile (J, J) read as its
  // P entry times its Q entry.
  template <bool KR = false>
  __device__ __forceinline__ void load(const T* __restrict__ yg, const T* __restrict__ cg,
                                       const T* __restrict__ lb, const T* __restrict__ ub, int64_t m,
                                       int64_t n, int64_t i0, int64_t j0, int64_t mat, const KronU& kr = KronU{}) {
    static_assert(!KR || sizeof(T) == 4, "Kronecker U: fp32");
    // the tile's corner in every operand (64-bit arithmetic once, uniform), then 32-bit offsets in
    // the tile (32 rows of at most 2^26 elements)
    const int rows_in = m - i0 < TR ? (int)(m - i0) : TR, cols_in = n - j0 < TR ? (int)(n - j0) : TR;
    const int ni = (int)n, mi = (int)m;
    const int64_t corner = i0 * n + j0;
    const T* yt = yg + mat + corner;
    const T* ct = cg + mat + corner;
    const T* lt = lb + i0 * m + i0;  // L[i0 + r, i0 + cc] at r m + cc
    const T* ut = KR ? nullptr : ub + j0 * n + j0;  // U[j0 + r, j0 + cc] at r n + cc
    T pu[NQ];  // KR: the P entries of the u[q]
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = threadIdx.x + NTHREADS * q;
      const int r = t / TR, cc = t % TR;
      const bool in = r < rows_in && cc < cols_in;
      const int off = r * ni + cc;
      y[q] = in ? yt[off] : T(0);
      c[q] = in ? ct[off] : T(0);
      // L[i0+r, i0+cc] strictly below the diagonal; U[j0+r, j0+cc] strictly above it
      l[q] = (cc < r && r < rows_in) ? lt[r * mi + cc] : T(0);
      if constexpr (KR) {
        const bool on = !ROWS && r < cc && cc < cols_in;
        int ib = 0, iq = 0, jb = 0, jq = 0;
        if (on) {
          kron_index(kr, (int)j0 + r, ib, iq);
          kron_index(kr, (int)j0 + cc, jb, jq);
        }
        u[q] = on ? kr.q[(int64_t)iq * kr.nq + jq] : T(0);
        pu[q] = on ? kr.p[(int64_t)ib * kr.np + jb] : T(0);
      } else {
        u[q] = (!ROWS && r < cc && cc < cols_in) ? ut[off] : T(0);
      }
    }
    if constexpr (KR) {  // the products after all loads (masked entries: 0 times 0)
#pragma unroll
      for (int q = 0; q < NQ; ++q) u[q] *= pu[q];
    }
  }

  // LDS image of the tile with the pulled feedback D (down) and R (right) added: C + D, Y + (D + R),
  // the zero padding of the diagonal blocks and of the C image, and the zeroed E image.  fp32: red holds
  // the waves' partial sums when `pulled` (pulled_sums: the first wd waves' are D's).  fp64: red64, when
  // given, holds D (red64[0]) and R (red64[1]) whole.
  __device__ __forceinline__ void store(TileLdsT<T>& tl, const float (*red)[2][TR][TR + 1], bool pulled, int wd,
                                        const double (*red64)[TR][TR + 1] = nullptr) const {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int t = threadIdx.x + NTHREADS * q;
      const int r = t / TR, cc = t % TR;
      T dd = T(0), rr = T(0);
      if constexpr (sizeof(T) == 4) {
        if (pulled) pulled_sums(red, wd, r, cc, dd, rr);
      } else {
        if (red64) dd = red64[0][r][cc], rr = red64[1][r][cc];
      }
      tl.Ys[r][cc] = y[q] + (dd + rr);
      tl.Cs[r][TR + cc] = c[q] + dd;
      tl.Lp[r][TR + cc] = l[q];
      if constexpr (!ROWS) tl.Up[TR + r][cc] = u[q];
    }
    if constexpr (ROWS) return;
    // zero padding without divisions: 8 threads per row of Lp and of Cs (71 and 66 padding columns), 4 per
    // padding row of Up (39 columns each); a strided column walk per thread
    {
      static_assert(NTHREADS == 8 * TR && LPW - TR <= 72 && CPW - TR <= 72 && UPW <= 40, "padding walk shape");
      const int r = threadIdx.x >> 3, sub = threadIdx.x & 7;
#pragma unroll
      for (int i = 0; i < 9; ++i) {
        const int k = sub + 8 * i;
        if (k < LPW - TR) tl.Lp[r][k < TR ? k : k + TR] = T(0);
        if (k < CPW - TR) tl.Cs[r][k < TR ? k : k + TR] = T(0);
      }
      const int row = threadIdx.x >> 2, sub4 = threadIdx.x & 3;
      T* up_row = tl.Up[row < TR ? row : row + TR];
#pragma unroll
      for (int i = 0; i < 10; ++i) {
        const int col = sub4 + 4 * i;
        if (col < UPW) up_row[col] = T(0);
      }
    }
    // the E image: all zeros (read times zero coefficients before the entries' errors are written)
    {
      T* es = &tl.Es[0][0];
      constexpr int EN = EROWS * SP;
#pragma unroll
      for (int i = 0; i < (EN + NTHREADS - 1) / NTHREADS; ++i) {
        const int k = threadIdx.x + NTHREADS * i;
        if (k < EN) es[k] = T(0);
      }
    }
  }
};

// A wave's partial product into red[product][half] (layout of the 32 x 32 MFMA accumulator).
__device__ __forceinline__ void stash_partial(float (*red)[2][TR][TR + 1], const floatx16& acc, int product,
                                              int half) {
  const int lane = threadIdx.x & 63, li = lane & 31, hh = lane >> 5;
#pragma unroll
  for (int r = 0; r < 16; ++r) red[product][half][8 * (r >> 2) + 4 * hh + (r & 3)][li] = acc[r];
}

// One launch per coarse stage T of the fused fp32 sweep, inside the outer block of tile stages
// [S0, S1).  The feedback a tile (I, J) needs from the tiles of its outer block swept before it
// (no flush has delivered it yet) is D = sum L[I,t] E[t,J] over t in [max(0, S0-J), I) and
// R = sum C[I,t] U[t,J] over t in [max(0, S0-I), J).  It is pulled on MFMA in two parts:
//  * prep workgroups (blockIdx.x >= n_sweep) take the tiles of stage T+1 and add the part from
//    the k-tiles before the last one (t < I-1, resp. t < J-1: stages up to T-1, all final) to
//    their Y and C in global memory -- no tile of stage T touches those;
//  * sweep workgroups take the tiles of stage T, pull the last k-tile (the tiles (I-1, J) and
//    (I, J-1) of stage T-1) and sweep the tile's 63 antidiagonals in LDS (sweep_tile).
// So only one k-tile of each product is on the stage-to-stage critical path; the rest runs beside
// the previous stage's sweeps.  Waves 0-1 take the down product, waves 2-3 the right one, each
// every second 8-deep k-chunk; the two halves meet in LDS.
// KR: U = P (x) Q given by its factors (kr; u unused): the right products pull Q times P entries.
template <bool VEC, int KIND, bool YPRE, bool ROWS, bool KR = false>
__global__ __launch_bounds__(NTHREADS, 2) void tile_stage_kernel(float* __restrict__ y, float* __restrict__ c,
                                                                 float* __restrict__ e, const float* __restrict__ l,
                                                                 const float* __restrict__ u, int64_t m, int64_t n,
                                                                 int64_t stage, int64_t S0, int64_t tile_lo,
                                                                 int64_t n_sweep, int64_t prep_lo, BatchMap lmap,
                                                                 BatchMap umap, QSpec<float> qs, int64_t nx,
                                                                 int64_t ny, KronU kr) {
  __shared__ float red[2][2][TR][TR + 1];
  __shared__ TileLds tl;

  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const bool sweep = id.x < n_sweep;
  const int64_t st = sweep ? stage : stage + 1;
  const int64_t I = sweep ? tile_lo + id.x : prep_lo + (id.x - n_sweep), J = st - I;
  const int64_t i0 = I * TR, j0 = J * TR;
  const int64_t mat = b * m * n;
  const float* lb = l + lmap.offset(b);
  const float* ub = KR ? nullptr : u + umap.offset(b);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hh = lane >> 5;

  // k-chunk ranges (8 columns each) of this workgroup's part of the two products
  const int64_t dlo = S0 - J > 0 ? S0 - J : 0, rlo = S0 - I > 0 ? S0 - I : 0;
  int64_t d0, d1, r0, r1;
  if (sweep) {
    d0 = I - 1 >= dlo ? 4 * (I - 1) : 0, d1 = I - 1 >= dlo ? 4 * I : 0;
    r0 = J - 1 >= rlo ? 4 * (J - 1) : 0, r1 = J - 1 >= rlo ? 4 * J : 0;
  } else {
    d0 = 4 * dlo, d1 = I - 1 > dlo ? 4 * (I - 1) : d0;
    r0 = 4 * rlo, r1 = J - 1 > rlo ? 4 * (J - 1) : r0;
  }
  const bool pulled = d0 < d1 || r0 < r1;
  if (!sweep && !pulled) return;

  // own tile data first: it does not depend on the pull, so its loads overlap the pull's
  TileRegs<ROWS> own;
  SweepInputs<ROWS ? Q_ROUND : KIND> qin;
  RowInputs<float, ROWS ? KIND : Q_ROUND> rin;
  if (sweep) {
    own.template load<KR>(y, c, lb, ub, m, n, i0, j0, mat, kr);
    if constexpr (ROWS)
      rin.load(qs, b, m, n, i0, j0);
    else
      qin.load(qs, b, m, n, i0, j0);
  }

  // the four waves dealt to the two products in proportion to their chunk counts (a tile near its
  // outer block's edge has nearly all its history in one of them), each product's chunks
  // interleaved over its waves
  const int64_t nd = d1 - d0, nr = r1 - r0;
  int wd = nd == 0 ? 0 : (nr == 0 ? 4 : (int)((4 * nd + (nd + nr) / 2) / (nd + nr)));
  if (nd > 0 && nr > 0) wd = wd < 1 ? 1 : (wd > 3 ? 3 : wd);
  if (pulled) {
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    if (wave < wd)
      pull_chunks<VEC>(acc, lb, m, m, m, e + mat, n, m, n, i0, j0, d0, d1, wave, wd, li, hh);
    else if constexpr (KR)
      pull_chunks_kron<VEC>(acc, c + mat, n, m, n, kr, n, n, i0, j0, r0, r1, wave - wd, 4 - wd, li, hh);
    else
      pull_chunks<VEC>(acc, c + mat, n, m, n, ub, n, n, n, i0, j0, r0, r1, wave - wd, 4 - wd, li, hh);
    stash_partial(red, acc, wave >> 1, wave & 1);
  }
  __syncthreads();

  if (!sweep) {  // prep: Y += D + R, C += D in place
    const int rows_in = m - i0 < TR ? (int)(m - i0) : TR, cols_in = n - j0 < TR ? (int)(n - j0) : TR;
    float* yt = y + mat + i0 * n + j0;
    float* ct = c + mat + i0 * n + j0;
#pragma unroll
    for (int q = 0; q < TR * TR / NTHREADS; ++q) {
      const int t = tid + NTHREADS * q;
      const int r = t / TR, cc = t % TR;
      if (r < rows_in && cc < cols_in) {
        const int off = r * (int)n + cc;
        float dd, rr;
        pulled_sums(red, wd, r, cc, dd, rr);
        yt[off] = yt[off] + (dd + rr);
        ct[off] = ct[off] + dd;
      }
    }
    return;
  }

  // ---- the tile image in LDS, then the in-tile sweep
  own.store(tl, red, pulled, wd);
  __syncthreads();
  if constexpr (ROWS)
    sweep_rows<float, KIND, YPRE>(&tl.Ys[0][0], SP, &tl.Cs[0][TR], CPW, &tl.Lp[0][TR], LPW, &tl.Es[TR][0], SP, rin, y, c,
                                  e, qs, m, n, i0, j0, mat);
  else
    sweep_tile<KIND, YPRE>(tl, qin, y, c, e, qs, m, n, i0, j0, mat);
}

// fp64 feedback of tile (I, J) from the k-tiles t in [d0, d1) (down: D = sum L[I,t] E[t,J]) and [r0, r1) (right:
// R = sum C[I,t] U[t,J]), on MFMA (v_mfma_f64_16x16x4_f64), into red[0] (D) and red[1] (R).  Wave w owns the
// 16 x 16 quadrant (w / 2, w % 2) of both products; lane l (q = l % 16, h = l / 16) supplies A(q, 8 h + s) and
// B(8 h + s, q) to MFMA s = 0..7 of a k-tile (which k a slot carries is free as long as A and B agree), and
// accumulator element r of lane l holds (h + 4 r, q) of the quadrant.  The k-tiles of both products form one
// list of jobs (D's first), loaded PJ jobs at a time, one chunk ahead of the chunk whose MFMAs run.
__device__ __forceinline__ void pull64(double (*red)[TR][TR + 1], const double* __restrict__ lb,
                                       const double* __restrict__ eb, const double* __restrict__ cb,
                                       const double* __restrict__ ub, int64_t m, int64_t n, int64_t i0, int64_t j0,
                                       int d0, int d1, int r0, int r1) {
  typedef double doublex4 __attribute__((ext_vector_type(4)));
  constexpr int PJ = 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 15, h = lane >> 4;
  const int64_t i = i0 + 16 * (wave >> 1) + q, j = j0 + 16 * (wave & 1) + q;
  const bool iin = i < m, jin = j < n;
  // this lane's rows of L and C, columns of E and U (64-bit arithmetic once)
  const double* la = lb + (iin ? i : 0) * m;
  const double* ca = cb + (iin ? i : 0) * n;
  const double* ej = eb + (jin ? j : 0);
  const double* uj = ub + (jin ? j : 0);
  const int nd = d1 - d0, nj = nd + (r1 - r0);
  double a[2][PJ][8], bv[2][PJ][8];
  // job x's operands: k = 32 t + 8 h + s, inside k < m (L's columns, E's rows) or k < n (C's columns, U's rows)
  auto load = [&](int x, double (&av)[8], double (&bb)[8]) {
    const bool dn = x < nd;
    const int64_t k0 = (int64_t)(dn ? d0 + x : r0 + (x - nd)) * TR + 8 * h;
    const int64_t kmax = dn ? m : n;
    const double* ap = dn ? la : ca;
    const double* bp = dn ? ej : uj;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bool ok = x < nj && k0 + s < kmax;
      av[s] = ok && iin ? ap[k0 + s] : 0.;
      bb[s] = ok && jin ? bp[(k0 + s) * n] : 0.;
    }
  };
  doublex4 accd = {0., 0., 0., 0.}, accr = {0., 0., 0., 0.};
  auto chunk = [&](int c0, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    if (c0 + PJ < nj) {
#pragma unroll
      for (int x = 0; x < PJ; ++x) load(c0 + PJ + x, a[1 - cur][x], bv[1 - cur][x]);
    }
#pragma unroll
    for (int x = 0; x < PJ; ++x) {
      const int job = c0 + x;  // uniform
      if (job >= nj) break;
      if (job < nd) {
#pragma unroll
        for (int s = 0; s < 8; ++s) accd = __builtin_amdgcn_mfma_f64_16x16x4f64(a[cur][x][s], bv[cur][x][s], accd, 0, 0, 0);
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) accr = __builtin_amdgcn_mfma_f64_16x16x4f64(a[cur][x][s], bv[cur][x][s], accr, 0, 0, 0);
      }
    }
  };
#pragma unroll
  for (int x = 0; x < PJ; ++x) load(x, a[0][x], bv[0][x]);
  for (int c0 = 0; c0 < nj; c0 += 2 * PJ) {
    chunk(c0, std::integral_constant<int, 0>{});
    if (c0 + PJ < nj) chunk(c0 + PJ, std::integral_constant<int, 1>{});
  }
  const int rq = 16 * (wave >> 1) + h, cq = 16 * (wave & 1) + q;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    red[0][rq + 4 * r][cq] = accd[r];
    red[1][rq + 4 * r][cq] = accr[r];
  }
}

// One launch per coarse stage of the fused fp64 sweep: each workgroup takes one tile of the stage.  Its
// feedback from the outer blocks before its own and from its own block's stages before `band_lo` has been
// flushed into its Y and C (outer flushes, then band flushes of `band` stages inside an outer block); the rest,
// from the tiles of stages [band_lo, stage), it pulls itself on MFMA (pull64).  Then it builds the fp32 sweep's
// LDS image in fp64 and runs the same push-form sweep of its 63 antidiagonals (sweep_tile).  The image and the
// pulled sums take 139 KB of LDS: one workgroup per CU, at most one per tile of the stage.
template <int KIND, bool YPRE>
__global__ __launch_bounds__(NTHREADS) void sweep_tile64_kernel(double* __restrict__ y, double* __restrict__ c,
                                                                double* __restrict__ e, const double* __restrict__ l,
                                                                const double* __restrict__ u, int64_t m, int64_t n,
                                                                int64_t stage, int64_t tile_lo, int64_t band_lo,
                                                                BatchMap lmap, BatchMap umap, QSpec<double> qs,
                                                                int64_t nx, int64_t ny) {
  __shared__ TileLdsT<double> tl;
  __shared__ double red[2][TR][TR + 1];
  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t I = tile_lo + id.x, J = stage - I;
  const int64_t i0 = I * TR, j0 = J * TR;
  const int64_t mat = b * m * n;
  const double* lb = l + lmap.offset(b);
  const double* ub = u + umap.offset(b);
  // k-tiles of the pull: the tiles (t, J) and (I, t) of stages [band_lo, stage)
  const int64_t dlo = band_lo - J > 0 ? band_lo - J : 0, rlo = band_lo - I > 0 ? band_lo - I : 0;
  const int d0 = (int)dlo, d1 = (int)(I > dlo ? I : dlo), r0 = (int)rlo, r1 = (int)(J > rlo ? J : rlo);
  const bool pulled = d0 < d1 || r0 < r1;
  SweepInputs<KIND, double> in;
  in.load(qs, b, m, n, i0, j0);
  TileRegs<false, double> regs;
  regs.load(y, c, lb, ub, m, n, i0, j0, mat);  // own data first: its loads overlap the pull's
  if (pulled) {
    pull64(red, lb, e + mat, c + mat, ub, m, n, i0, j0, d0, d1, r0, r1);
    __syncthreads();
  }
  regs.store(tl, nullptr, false, 0, pulled ? red : nullptr);
  __syncthreads();
  sweep_tile<KIND, YPRE>(tl, in, y, c, e, qs, m, n, i0, j0, mat);
}

template <int KIND>
void launch_tile64_k(dim3 grid, hipStream_t stream, double* y, double* c, double* e, const double* l, const double* u,
                     int64_t m, int64_t n, int64_t st, int64_t lo, int64_t band_lo, const BatchMap& lmap,
                     const BatchMap& umap, const QSpec<double>& qs, int64_t nx, int64_t ny) {
  if (qs.ypre)
    hipLaunchKernelGGL((sweep_tile64_kernel<KIND, true>), grid, dim3(NTHREADS), 0, stream, y, c, e, l, u, m, n, st, lo,
                       band_lo, lmap, umap, qs, nx, ny);
  else
    hipLaunchKernelGGL((sweep_tile64_kernel<KIND, false>), grid, dim3(NTHREADS), 0, stream, y, c, e, l, u, m, n, st,
                       lo, band_lo, lmap, umap, qs, nx, ny);
}

template <bool VEC, int KIND, bool ROWS, bool KR>
void launch_tile_stage_k(dim3 grid, hipStream_t stream, float* y, float* c, float* e, const float* l, const float* u,
                         int64_t m, int64_t n, int64_t st, int64_t S0, int64_t lo, int64_t n_sweep, int64_t prep_lo,
                         const BatchMap& lmap, const BatchMap& umap, const QSpec<float>& qs, int64_t nx, int64_t ny,
                         const KronU& kr) {
  if (qs.ypre)
    hipLaunchKernelGGL((tile_stage_kernel<VEC, KIND, true, ROWS, KR>), grid, dim3(NTHREADS), 0, stream, y, c, e, l, u,
                       m, n, st, S0, lo, n_sweep, prep_lo, lmap, umap, qs, nx, ny, kr);
  else
    hipLaunchKernelGGL((tile_stage_kernel<VEC, KIND, false, ROWS, KR>), grid, dim3(NTHREADS), 0, stream, y, c, e, l, u,
                       m, n, st, S0, lo, n_sweep, prep_lo, lmap, umap, qs, nx, ny, kr);
}

template <bool VEC, bool ROWS, bool KR = false>
void launch_tile_stage(int32_t kind, dim3 grid, hipStream_t stream, float* y, float* c, float* e, const float* l,
                       const float* u, int64_t m, int64_t n, int64_t st, int64_t S0, int64_t lo, int64_t n_sweep,
                       int64_t prep_lo, const BatchMap& lmap, const BatchMap& umap, const QSpec<float>& qs, int64_t nx,
                       int64_t ny, const KronU& kr = KronU{}) {
  if (kind == Q_AFFINE)
    launch_tile_stage_k<VEC, Q_AFFINE, ROWS, KR>(grid, stream, y, c, e, l, u, m, n, st, S0, lo, n_sweep, prep_lo, lmap,
                                                 umap, qs, nx, ny, kr);
  else if (kind == Q_FORCED)
    launch_tile_stage_k<VEC, Q_FORCED, ROWS, KR>(grid, stream, y, c, e, l, u, m, n, st, S0, lo, n_sweep, prep_lo, lmap,
                                                 umap, qs, nx, ny, kr);
  else if (ROWS && kind == Q_ABSMAX)
    launch_tile_stage_k<VEC, Q_ABSMAX, true, KR>(grid, stream, y, c, e, l, u, m, n, st, S0, lo, n_sweep, prep_lo, lmap,
                                                 umap, qs, nx, ny, kr);
  else
    launch_tile_stage_k<VEC, Q_ROUND, ROWS, KR>(grid, stream, y, c, e, l, u, m, n, st, S0, lo, n_sweep, prep_lo, lmap,
                                                umap, qs, nx, ny, kr);
}

template <typename T, int KIND>
void launch_rows_stage(dim3 grid, hipStream_t stream, T* y, T* c, T* e, const T* l, int64_t m, int64_t n, int64_t st,
                       int64_t lo, const BatchMap& lmap, const QSpec<T>& qs, int64_t nx, int64_t ny) {
  if (qs.ypre)
    hipLaunchKernelGGL((sweep_rows_kernel<T, KIND, true>), grid, dim3(NTHREADS), 0, stream, y, c, e, l, m, n, st, lo,
                       lmap, qs, nx, ny);
  else
    hipLaunchKernelGGL((sweep_rows_kernel<T, KIND, false>), grid, dim3(NTHREADS), 0, stream, y, c, e, l, m, n, st, lo,
                       lmap, qs, nx, ny);
}

bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15) == 0; }

bool strides_mult4(const BatchMap& bm) {
  for (int d = 0; d < bm.nd; ++d)
    if (bm.stride[d] % 4) return false;
  return true;
}

// rows: super-entries of 1 x TR (the row sweep); dtype16: the abs-max scale's 16-bit type; kron: U given by its
// Kronecker factors (u unused; fp32, one matrix, rows staged 128 bits at a time).
template <typename T>
int sweep_fused(T* y, T* c, T* e, const T* l, const T* u, int64_t m, int64_t n, int32_t bnd, const int64_t* bshape,
                const int64_t* lstride, const int64_t* ustride, int32_t qkind, const T* qa, const int64_t* qa_stride,
                const T* qb, const int64_t* qb_stride, double qmin, double qmax, T* ypre, int64_t outer_tiles,
                int64_t stage_begin, int64_t stage_end, hipStream_t stream, bool rows = false, int32_t dtype16 = 0,
                T* scale_out = nullptr, const KronU* kron = nullptr) {
  BatchMap lmap, umap;
  if (!make_batch_map(lmap, bnd, bshape, lstride) || !make_batch_map(umap, bnd, bshape, ustride)) return GPTQ2D_EINVAL;
  if (m <= 0 || n <= 0 || outer_tiles < 1) return GPTQ2D_EINVAL;
  // U from its factors: the outer flush that reads them is the tuned tile flush alone (m, n < 2^20), so sizes it
  // rejects are refused here, before any stage has written y
  if (kron && (sizeof(T) != 4 || bnd != 0 || n != (int64_t)kron->np * kron->nq || m >= ((int64_t)1 << 20) ||
               n >= ((int64_t)1 << 20)))
    return GPTQ2D_EUNSUPPORTED;
  // the tile kernels index inside a tile with 32-bit offsets (32 rows of a row length < 2^26)
  if (m >= ((int64_t)1 << 26) || n >= ((int64_t)1 << 26)) return GPTQ2D_EUNSUPPORTED;
  if (qkind != Q_ROUND && qkind != Q_AFFINE && qkind != Q_FORCED && !(rows && qkind == Q_ABSMAX)) return GPTQ2D_EINVAL;
  if ((qkind == Q_AFFINE && (!qa || !qb)) || (qkind == Q_FORCED && !qa)) return GPTQ2D_EINVAL;
  if (qkind == Q_ABSMAX && (!(qmin < qmax) || (dtype16 != 1 && dtype16 != 2))) return GPTQ2D_EINVAL;
  if (rows && n % TR) return GPTQ2D_EINVAL;  // the super-entries tile the rows
  QSpec<T> qs;
  qs.kind = qkind;
  qs.scale = qa;
  qs.zp = qb;
  if (!make_batch_map(qs.smap, bnd, bshape, qa_stride) || !make_batch_map(qs.zmap, bnd, bshape, qb_stride))
    return GPTQ2D_EINVAL;
  qs.qmin = (T)qmin;
  qs.qmax = (T)qmax;
  qs.ypre = ypre;
  qs.sout = qkind == Q_ABSMAX ? scale_out : nullptr;
  qs.dtype16 = dtype16;
  const int64_t B = batch_count(bnd, bshape);
  if (B == 0) return 0;
  const int64_t mt = cdiv(m, TR), nt = cdiv(n, TR), stages = mt + nt - 1;
  if (stage_end < 0 || stage_end > stages) stage_end = stages;
  // a call covers whole outer blocks: [stage_begin, stage_end) starts on an outer block's first stage and
  // ends after one's last (or at the end of the sweep), so that consecutive calls resume exactly
  if (stage_begin < 0 || stage_begin > stage_end || stage_begin % outer_tiles ||
      (stage_end % outer_tiles && stage_end != stages))
    return GPTQ2D_EINVAL;
  // 128-bit operand loads of the MFMA pull: rows, matrices and pointers 16-byte aligned
  const bool vec = m % 4 == 0 && n % 4 == 0 && aligned16(y) && aligned16(c) && aligned16(e) && aligned16(l) &&
                   aligned16(u) && strides_mult4(lmap) && strides_mult4(umap);
  if (kron && !(vec && aligned16(kron->q))) return GPTQ2D_EUNSUPPORTED;
  int rc;
  if (stage_begin == 0 && (rc = gptq2d_fill<T>(c, T(0), B * m * n, stream))) return rc;
  // fp64: stages per band flush inside an outer block (the tile sweeps pull the band's earlier stages); the row
  // sweep pulls nothing, so its every stage is flushed
  const int64_t band = rows ? 1 : BAND64;
  for (int64_t S0 = stage_begin; S0 < stage_end; S0 += outer_tiles) {
    const int64_t S1 = S0 + outer_tiles < stages ? S0 + outer_tiles : stages;
    for (int64_t st = S0; st < S1; ++st) {
      const int64_t lo = st - nt + 1 > 0 ? st - nt + 1 : 0;
      const int64_t hi = st < mt - 1 ? st : mt - 1;
      const bool prof = gptq2d_prof_on(PROF_TILE_SWEEP);
      if (prof) gptq2d_prof_begin(PROF_TILE_SWEEP, stream);
      if constexpr (sizeof(T) == 4) {
        // fp32: this stage's sweeps plus the prep of the next stage of the outer block
        int64_t plo = 0, pcount = 0;
        if (st + 1 < S1) {
          plo = st + 1 - nt + 1 > 0 ? st + 1 - nt + 1 : 0;
          pcount = (st + 1 < mt - 1 ? st + 1 : mt - 1) - plo + 1;
        }
        const Grid3 g = make_grid(hi - lo + 1 + pcount, 1, B);
        auto launch = [&](auto vec_c, auto rows_c) {
          launch_tile_stage<decltype(vec_c)::value, decltype(rows_c)::value>(
              qkind, g.grid, stream, y, c, e, l, u, m, n, st, S0, lo, hi - lo + 1, plo, lmap, umap, qs, g.nx, g.ny);
        };
        using True = std::true_type;
        using False = std::false_type;
        if (kron) {
          if (rows)
            launch_tile_stage<true, true, true>(qkind, g.grid, stream, y, c, e, l, nullptr, m, n, st, S0, lo,
                                                hi - lo + 1, plo, lmap, umap, qs, g.nx, g.ny, *kron);
          else
            launch_tile_stage<true, false, true>(qkind, g.grid, stream, y, c, e, l, nullptr, m, n, st, S0, lo,
                                                 hi - lo + 1, plo, lmap, umap, qs, g.nx, g.ny, *kron);
        } else if (vec)
          rows ? launch(True{}, True{}) : launch(True{}, False{});
        else
          rows ? launch(False{}, True{}) : launch(False{}, False{});
      } else {
        const Grid3 g = make_grid(hi - lo + 1, 1, B);
        if (rows) {
          if (qkind == Q_AFFINE)
            launch_rows_stage<T, Q_AFFINE>(g.grid, stream, y, c, e, l, m, n, st, lo, lmap, qs, g.nx, g.ny);
          else if (qkind == Q_FORCED)
            launch_rows_stage<T, Q_FORCED>(g.grid, stream, y, c, e, l, m, n, st, lo, lmap, qs, g.nx, g.ny);
          else if (qkind == Q_ABSMAX)
            launch_rows_stage<T, Q_ABSMAX>(g.grid, stream, y, c, e, l, m, n, st, lo, lmap, qs, g.nx, g.ny);
          else
            launch_rows_stage<T, Q_ROUND>(g.grid, stream, y, c, e, l, m, n, st, lo, lmap, qs, g.nx, g.ny);
        } else {
          // the push-form sweep of the fp32 engine, in fp64, pulling its band's earlier stages
          const int64_t blo = st - (st - S0) % band;
          if (qkind == Q_AFFINE)
            launch_tile64_k<Q_AFFINE>(g.grid, stream, y, c, e, l, u, m, n, st, lo, blo, lmap, umap, qs, g.nx, g.ny);
          else if (qkind == Q_FORCED)
            launch_tile64_k<Q_FORCED>(g.grid, stream, y, c, e, l, u, m, n, st, lo, blo, lmap, umap, qs, g.nx, g.ny);
          else
            launch_tile64_k<Q_ROUND>(g.grid, stream, y, c, e, l, u, m, n, st, lo, blo, lmap, umap, qs, g.nx, g.ny);
        }
      }
      // work of a tile sweep: its entries (the in-tile feedback is latency-, not throughput-bound)
      if (prof) gptq2d_prof_end(PROF_TILE_SWEEP, (double)B * (hi - lo + 1) * TR * TR, stream);
      if ((rc = (int)hipGetLastError())) return rc;
      if constexpr (sizeof(T) == 8) {
        // a band's stages into the rest of the outer block, after the band's last stage
        if (st + 1 < S1 && (st + 1 - S0) % band == 0 &&
            (rc = gptq2d_flush<T>(y, c, e, l, u, m, n, TR, TR, st + 1 - band, st + 1, S1, lmap, umap, B, stream)))
          return rc;
      }
    }
    if (S1 < stages) {
      if constexpr (sizeof(T) == 4) {
        if (kron) {
          if ((rc = gptq2d_flush_kron(y, c, e, l, *kron, m, n, S0, S1, stages, stream))) return rc;
          continue;
        }
      }
      if ((rc = gptq2d_flush<T>(y, c, e, l, u, m, n, TR, TR, S0, S1, stages, lmap, umap, B, stream))) return rc;
    }
  }
  return 0;
}

// ------------------------------------------------------------------------------------------------ no-alloc entry

// Scratch of gptq2d_sweep_fused_noalloc_*: the sweep's C and E buffers, each half of this array, in a
// fixed device array that the HIP runtime places on every GPU that loads the library (it stays there
// until the process ends).  Host code never uses the name `scratch` as an address (it is a host-side
// stand-in): the device address comes from hipGetSymbolAddress, once per device, on the first call
// made with that device current.
constexpr int64_t NOALLOC_SCRATCH_BYTES = (int64_t)128 << 20;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex scratch_mutex;
void* scratch_ptr[NOALLOC_MAX_DEVICES];

// Device address of the current device's scratch array, or nullptr if it cannot be had.
void* scratch_address() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) return nullptr;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    scratch_ptr[dev] = p;
  }
  return scratch_ptr[dev];
}

template <typename T>
int sweep_fused_noalloc(T* y, const T* l, const T* u, int64_t m, int64_t n, int32_t bnd, const int64_t* bshape,
                        const int64_t* lstride, const int64_t* ustride, int32_t qkind, const T* qa,
                        const int64_t* qa_stride, const T* qb, const int64_t* qb_stride, double qmin, double qmax,
                        T* ypre, int64_t outer_tiles, hipStream_t stream) {
  if (m < 0 || n < 0 || bnd < 0 || bnd > GPTQ2D_MAX_BATCH_DIMS) return GPTQ2D_EINVAL;
  // each of C and E takes half the array: B m n elements of T at most (checked before any product can
  // overflow: every factor is below 2^31 once the first test passes)
  const int64_t cap = NOALLOC_SCRATCH_BYTES / 2 / (int64_t)sizeof(T);
  int64_t count = 1;
  for (int32_t d = 0; d < bnd; ++d) {
    if (bshape[d] < 0) return GPTQ2D_EINVAL;
    count = bshape[d] == 0 || count == 0 ? 0 : (bshape[d] > cap / count ? cap + 1 : count * bshape[d]);
  }
  if (m > 0 && n > 0 && count > 0 && (m > cap || n > cap / m || count > cap / (m * n))) return GPTQ2D_ESCRATCH;
  T* c = static_cast<T*>(scratch_address());
  if (!c) return GPTQ2D_EUNSUPPORTED;
  T* e = c + cap;
  return sweep_fused<T>(y, c, e, l, u, m, n, bnd, bshape, lstride, ustride, qkind, qa, qa_stride, qb, qb_stride, qmin,
                        qmax, ypre, outer_tiles, 0, -1, stream);
}

}  // namespace

extern "C" {

#define GPTQ2D_FUSED_ABI(SUF, T)                                                                                    \
  int gptq2d_sweep_fused_##SUF(T* y, T* c, T* e, const T* l, const T* u, int64_t m, int64_t n, int32_t bnd,        \
                               const int64_t* bshape, const int64_t* lstride, const int64_t* ustride, int32_t qkind, \
                               const T* qa, const int64_t* qa_stride, const T* qb, const int64_t* qb_stride,       \
                               double qmin, double qmax, T* ypre, int64_t outer_tiles, int64_t stage_begin,          \
                               int64_t stage_end, hipStream_t stream) {                                              \
    return sweep_fused<T>(y, c, e, l, u, m, n, bnd, bshape, lstride, ustride, qkind, qa, qa_stride, qb, qb_stride,   \
                          qmin, qmax, ypre, outer_tiles, stage_begin, stage_end, stream);                             \
  }                                                                                                                  \
  int64_t gptq2d_sweep_fused_tile_##SUF(void) { return TR; }                                                      \
  int gptq2d_sweep_fused_se_##SUF(T* y, T* c, T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t p,         \
                                  int64_t q, int32_t bnd, const int64_t* bshape, const int64_t* lstride,             \
                                  const int64_t* ustride, int32_t qkind, const T* qa, const int64_t* qa_stride,     \
                                  const T* qb, const int64_t* qb_stride, double qmin, double qmax, int32_t dtype16, \
                                  T* ypre, T* scale_out, int64_t outer_tiles, int64_t stage_begin,                  \
                                  int64_t stage_end, hipStream_t stream) {                                           \
    if (p <= 0 || q <= 0 || m % p || n % q) return GPTQ2D_EINVAL;                                                  \
    if (p == 1 && q == 1 && qkind != Q_ABSMAX)                                                                       \
      return sweep_fused<T>(y, c, e, l, u, m, n, bnd, bshape, lstride, ustride, qkind, qa, qa_stride, qb, qb_stride, \
                            qmin, qmax, ypre, outer_tiles, stage_begin, stage_end, stream);                          \
    if (p != 1 || q != TR) return GPTQ2D_EUNSUPPORTED;                                                              \
    return sweep_fused<T>(y, c, e, l, u, m, n, bnd, bshape, lstride, ustride, qkind, qa, qa_stride, qb, qb_stride,   \
                          qmin, qmax, ypre, outer_tiles, stage_begin, stage_end, stream, true, dtype16, scale_out);  \
  }                                                                                                                  \
  int gptq2d_sweep_fused_noalloc_##SUF(T* y, const T* l, const T* u, int64_t m, int64_t n, int32_t bnd,              \
                                       const int64_t* bshape, const int64_t* lstride, const int64_t* ustride,       \
                                       int32_t qkind, const T* qa, const int64_t* qa_stride, const T* qb,           \
                                       const int64_t* qb_stride, double qmin, double qmax, T* ypre,                 \
                                       int64_t outer_tiles, hipStream_t stream) {                                    \
    return sweep_fused_noalloc<T>(y, l, u, m, n, bnd, bshape, lstride, ustride, qkind, qa, qa_stride, qb, qb_stride, \
                                  qmin, qmax, ypre, outer_tiles, stream);                                            \
  }

int64_t gptq2d_sweep_fused_noalloc_capacity(int32_t elem_bytes) {
  return elem_bytes == 4 || elem_bytes == 8 ? NOALLOC_SCRATCH_BYTES / 2 / elem_bytes : -1;
}

GPTQ2D_FUSED_ABI(f32, float)
GPTQ2D_FUSED_ABI(f64, double)

int gptq2d_sweep_fused_kron_f32(float* y, float* c, float* e, const float* l, const float* up, const float* uq,
                                int64_t m, int64_t np, int64_t nq, int64_t p, int64_t q, int32_t qkind,
                                const float* qa, const float* qb, double qmin, double qmax, int32_t dtype16,
                                float* ypre, float* scale_out, int64_t outer_tiles, int64_t stage_begin,
                                int64_t stage_end, hipStream_t stream) {
  if (!up || !uq || np <= 0 || nq <= 0 || p <= 0 || q <= 0) return GPTQ2D_EINVAL;
  KronU kr;
  if (!make_kron_u(kr, up, uq, np, nq)) return GPTQ2D_EUNSUPPORTED;
  const int64_t n = np * nq;
  if (m % p || n % q) return GPTQ2D_EINVAL;
  const bool rows = !(p == 1 && q == 1 && qkind != Q_ABSMAX);
  if (rows && (p != 1 || q != TR)) return GPTQ2D_EUNSUPPORTED;
  return sweep_fused<float>(y, c, e, l, nullptr, m, n, 0, nullptr, nullptr, nullptr, qkind, qa, nullptr, qb, nullptr,
                            qmin, qmax, ypre, outer_tiles, stage_begin, stage_end, stream, rows, dtype16, scale_out,
                            &kr);
}

}  // extern "C"
