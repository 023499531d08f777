// Fused GPTQ-2D sweep for per-entry quantizers (round, affine, teacher-forced codes).
//
// The matrix is cut into TR x TR tiles.  GPTQ-2D gives the same rounding for any order of the
// entries that respects the partial order (i' <= i, j' <= j), so the sweep runs over coarse
// stages T = I + J of tiles: the tiles of one coarse stage do not depend on each other, and each
// is swept by one workgroup entirely in LDS -- its 2*TR-1 antidiagonals one after another, every
// entry of an antidiagonal at once, the in-tile error feedback through the diagonal blocks
// L[I,I] and U[J,J], the quantizer applied in place.  Feedback between tiles is the block flush
// of flush.hip with P = Q = TR: after each coarse stage into the rest of its outer block, and after
// each outer block of `outer_tiles` coarse stages into all later stages.  The host loop below
// issues every launch of the sweep from C++ in one call, so a whole layer is one C-ABI call and
// one capturable stream of kernels.
//
// In exact arithmetic the result equals the reference's blocked sweep (gptq_2d.py:1295-1375) and
// Algorithm 1 on vec(X) (GPTQ-2D paper, Theorem 1); in floating point the sums are accumulated in
// a different order.  In-tile feedback of entry (r, c) is gathered ("pulled") as
//   y = (Y[r,c] + sum_{r'<r} L[r,r'] E[r',c]) + sum_{c'<c} C[r,c'] U[c',c]
// where C[r,c'] is already complete (all rows above in the tile were rounded earlier).
#include "common.h"
#include "profile.h"

template <typename T>
int gptq2d_flush(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t P, int64_t Q,
                 int64_t s0, int64_t s1, int64_t s_end, const BatchMap& lmap, const BatchMap& umap, int64_t B,
                 hipStream_t stream);
template <typename T>
int gptq2d_fill(T* x, T v, int64_t count, hipStream_t stream);

namespace {

constexpr int TR = 32;       // tile edge
constexpr int PARTS = 8;     // threads cooperating on one entry of an antidiagonal
constexpr int NTHREADS = TR * PARTS;

enum QKind : int32_t { Q_ROUND = 0, Q_AFFINE = 1, Q_FORCED = 2 };

template <typename T>
struct QSpec {
  int32_t kind;
  const T* scale;  // affine: full [*, m, n] scale; forced: the codes' values
  const T* zp;     // affine: full [*, m, n] zero point
  BatchMap smap, zmap;
  T qmin, qmax;
  T* ypre;  // optional [B, m, n]: Y of every entry just before it is rounded
};

template <typename T>
__global__ __launch_bounds__(NTHREADS) void sweep_tiles_kernel(T* __restrict__ y, T* __restrict__ c,
                                                               T* __restrict__ e, const T* __restrict__ l,
                                                               const T* __restrict__ u, int64_t m, int64_t n,
                                                               int64_t stage, int64_t tile_lo, BatchMap lmap,
                                                               BatchMap umap, QSpec<T> qs, int64_t nx, int64_t ny) {
  __shared__ T Ys[TR][TR + 1];
  __shared__ T Cs[TR][TR + 1];
  __shared__ T Es[TR][TR + 1];
  __shared__ T Ls[TR][TR + 1];
  __shared__ T Us[TR][TR + 1];
  __shared__ T Ss[TR][TR + 1];
  __shared__ T Zs[TR][TR + 1];

  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t I = tile_lo + id.x, J = stage - I;
  const int64_t i0 = I * TR, j0 = J * TR;
  const int64_t mat = b * m * n;
  const T* lb = l + lmap.offset(b);
  const T* ub = u + umap.offset(b);
  const int tid = threadIdx.x;

  for (int t = tid; t < TR * TR; t += NTHREADS) {
    const int r = t / TR, cc = t % TR;
    const int64_t gi = i0 + r, gj = j0 + cc;
    const bool in = gi < m && gj < n;
    const int64_t off = mat + gi * n + gj;
    Ys[r][cc] = in ? y[off] : T(0);
    Cs[r][cc] = in ? c[off] : T(0);
    Es[r][cc] = T(0);
    // L[i0+r, i0+cc] strictly below the diagonal; U[j0+r, j0+cc] strictly above it
    Ls[r][cc] = (cc < r && gi < m) ? lb[gi * m + (i0 + cc)] : T(0);
    Us[r][cc] = (r < cc && j0 + cc < n) ? ub[(j0 + r) * n + (j0 + cc)] : T(0);
    if (qs.kind == Q_AFFINE) {
      Ss[r][cc] = in ? qs.scale[qs.smap.offset(b) + gi * n + gj] : T(1);
      Zs[r][cc] = in ? qs.zp[qs.zmap.offset(b) + gi * n + gj] : T(0);
    } else if (qs.kind == Q_FORCED) {
      Ss[r][cc] = in ? qs.scale[qs.smap.offset(b) + gi * n + gj] : T(0);
    }
  }
  __syncthreads();

  const int r = tid / PARTS, part = tid % PARTS;
  const int64_t gi = i0 + r;
  for (int t = 0; t < 2 * TR - 1; ++t) {
    const int cc = t - r;
    const bool active = cc >= 0 && cc < TR && gi < m && j0 + cc < n;
    T down = T(0), right = T(0);
    if (active) {
#pragma unroll
      for (int k = 0; k < TR / PARTS; ++k) {
        const int rr = part + PARTS * k;
        if (rr < r) down += Ls[r][rr] * Es[rr][cc];
      }
#pragma unroll
      for (int k = 0; k < TR / PARTS; ++k) {
        const int c2 = part + PARTS * k;
        if (c2 < cc) right += Cs[r][c2] * Us[c2][cc];
      }
    }
#pragma unroll
    for (int w = PARTS / 2; w >= 1; w >>= 1) {
      down += __shfl_xor(down, w, PARTS);
      right += __shfl_xor(right, w, PARTS);
    }
    if (active && part == 0) {
      const T yv = (Ys[r][cc] + down) + right;
      T z;
      if (qs.kind == Q_AFFINE) {
        const T sv = Ss[r][cc], zv = Zs[r][cc];
        const T code = clamp_val(round_even(yv / sv + zv), qs.qmin, qs.qmax);
        z = (code - zv) * sv;
      } else if (qs.kind == Q_FORCED) {
        z = Ss[r][cc];
      } else {
        z = round_even(yv);
      }
      const T ev = z - yv;
      Ys[r][cc] = z;
      Es[r][cc] = ev;
      Cs[r][cc] = (Cs[r][cc] + down) + ev;
      if (qs.ypre) qs.ypre[mat + gi * n + j0 + cc] = yv;
    }
    __syncthreads();
  }

  for (int t = tid; t < TR * TR; t += NTHREADS) {
    const int rr = t / TR, cc = t % TR;
    const int64_t gi2 = i0 + rr, gj = j0 + cc;
    if (gi2 < m && gj < n) {
      const int64_t off = mat + gi2 * n + gj;
      y[off] = Ys[rr][cc];
      c[off] = Cs[rr][cc];
      e[off] = Es[rr][cc];
    }
  }
}

template <typename T>
int sweep_fused(T* y, T* c, T* e, const T* l, const T* u, int64_t m, int64_t n, int32_t bnd, const int64_t* bshape,
                const int64_t* lstride, const int64_t* ustride, int32_t qkind, const T* qa, const int64_t* qa_stride,
                const T* qb, const int64_t* qb_stride, double qmin, double qmax, T* ypre, int64_t outer_tiles,
                int64_t stage_begin, int64_t stage_end, hipStream_t stream) {
  BatchMap lmap, umap;
  if (!make_batch_map(lmap, bnd, bshape, lstride) || !make_batch_map(umap, bnd, bshape, ustride)) return GPTQ2D_EINVAL;
  if (m <= 0 || n <= 0 || outer_tiles < 1) return GPTQ2D_EINVAL;
  if (qkind != Q_ROUND && qkind != Q_AFFINE && qkind != Q_FORCED) return GPTQ2D_EINVAL;
  if ((qkind == Q_AFFINE && (!qa || !qb)) || (qkind == Q_FORCED && !qa)) return GPTQ2D_EINVAL;
  QSpec<T> qs;
  qs.kind = qkind;
  qs.scale = qa;
  qs.zp = qb;
  if (!make_batch_map(qs.smap, bnd, bshape, qa_stride) || !make_batch_map(qs.zmap, bnd, bshape, qb_stride))
    return GPTQ2D_EINVAL;
  qs.qmin = (T)qmin;
  qs.qmax = (T)qmax;
  qs.ypre = ypre;
  const int64_t B = batch_count(bnd, bshape);
  if (B == 0) return 0;
  const int64_t mt = cdiv(m, TR), nt = cdiv(n, TR), stages = mt + nt - 1;
  if (stage_end < 0 || stage_end > stages) stage_end = stages;
  if (stage_begin < 0 || stage_begin > stage_end || stage_begin % outer_tiles) return GPTQ2D_EINVAL;
  int rc;
  if (stage_begin == 0 && (rc = gptq2d_fill<T>(c, T(0), B * m * n, stream))) return rc;
  for (int64_t S0 = stage_begin; S0 < stage_end; S0 += outer_tiles) {
    const int64_t S1 = S0 + outer_tiles < stages ? S0 + outer_tiles : stages;
    for (int64_t st = S0; st < S1; ++st) {
      const int64_t lo = st - nt + 1 > 0 ? st - nt + 1 : 0;
      const int64_t hi = st < mt - 1 ? st : mt - 1;
      Grid3 g = make_grid(hi - lo + 1, 1, B);
      const bool prof = gptq2d_prof_on(PROF_TILE_SWEEP);
      if (prof) gptq2d_prof_begin(PROF_TILE_SWEEP, stream);
      hipLaunchKernelGGL(sweep_tiles_kernel<T>, g.grid, dim3(NTHREADS), 0, stream, y, c, e, l, u, m, n, st, lo, lmap,
                         umap, qs, g.nx, g.ny);
      // work of a tile sweep: its entries (the in-tile feedback is latency-, not throughput-bound)
      if (prof) gptq2d_prof_end(PROF_TILE_SWEEP, (double)B * (hi - lo + 1) * TR * TR, stream);
      if ((rc = (int)hipGetLastError())) return rc;
      if (st + 1 < S1 && (rc = gptq2d_flush<T>(y, c, e, l, u, m, n, TR, TR, st, st + 1, S1, lmap, umap, B, stream)))
        return rc;
    }
    if (S1 < stages && (rc = gptq2d_flush<T>(y, c, e, l, u, m, n, TR, TR, S0, S1, stages, lmap, umap, B, stream)))
      return rc;
  }
  return 0;
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
  int64_t gptq2d_sweep_fused_tile_##SUF(void) { return TR; }

GPTQ2D_FUSED_ABI(f32, float)
GPTQ2D_FUSED_ABI(f64, double)

}  // extern "C"
