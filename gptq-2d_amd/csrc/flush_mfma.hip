// Cross-tile flush of the fused sweep on fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// In the fused engine the stages are the coarse antidiagonals I + J of 32 x 32 tiles (P = Q = 32
// in flush.hip's terms), so every band boundary is a tile boundary and each 32 x 32 MFMA output
// block is exactly one target tile.  For the band of tile stages [S0, S1) and a target tile (I, J)
// with S1 <= I + J < S_end:
//
//   D(I,J) = sum_{t in [S0-J, S1-J), 0 <= t < I}  L[I, t] E[t, J]      (32 x 32 x 32 products)
//   R(I,J) = sum_{t in [S0-I, S1-I), 0 <= t < J}  C[I, t] U[t, J]
//   C[I,J] += D;   Y[I,J] += D + R
//
// A workgroup owns WT x WT target tiles and four waves, each wave (WT/2) x (WT/2) tiles with one
// 16-register accumulator per tile.  The K loop walks the union of the tiles' k-tile ranges; each
// k-tile's panels (A: the WG's rows x 32 of L, then of C; B: 32 x the WG's columns of E, then of U)
// are prefetched into registers with 128-bit loads one k-tile ahead and stored to LDS, and a wave
// issues a tile's 16 MFMAs only when the k-tile lies in that tile's own range -- no MFMA is spent
// on a masked zero, and tiles that receive nothing are not read or written.  Staging loads are
// masked to exactly the entries a product may read: L strictly below, U strictly above its
// diagonal tiles, E and C on the band, nothing outside the matrix.
//
// Operand layout (lane l, i = l % 32, h = l / 32): A(i, kslot = h), B(kslot = h, j = i); the 16
// accumulators hold D(8 (r / 4) + 4 h + r % 4, i).  The k carried by slot h in MFMA s is 16 h + s
// for both operands, so 16 MFMAs cover the 32-deep k-tile; A is read from LDS as four 128-bit loads
// of 16 consecutive k, B as 16 conflict-free 32-bit loads along j.
//
// Reference counterparts (IST-DASLab/GPTQ-2D, gptq_2d.py): _flush_down_kernel :766-932 and
// _flush_right_kernel :936-1087 (fp32 `tl.dot` with input_precision="ieee"); one kernel here, with
// one read-modify-write of Y and C per target tile.
#include "common.h"

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int TS = 32;      // tile edge = MFMA block edge
constexpr int AP = TS + 4;  // LDS pitch of the A panel rows (k fastest), 16-byte aligned

struct TileFlush {
  int64_t m, n, mt, nt, S0, S1, S_end;
};

__device__ __forceinline__ bool is_target(const TileFlush& g, int64_t I, int64_t J) {
  return I < g.mt && J < g.nt && I + J >= g.S1 && I + J < g.S_end;
}

// k-tile range of the down (phase 0) or right (phase 1) product of tile (I, J): [lo, hi)
__device__ __forceinline__ void tile_range(const TileFlush& g, int phase, int64_t I, int64_t J, int64_t& lo,
                                           int64_t& hi) {
  const int64_t a = phase == 0 ? J : I, b = phase == 0 ? I : J;
  lo = g.S0 - a > 0 ? g.S0 - a : 0;
  hi = g.S1 - a < b ? g.S1 - a : b;
}

template <int WT, bool VEC>
__global__ __launch_bounds__(256, 2) void flush_tiles_mfma_kernel(float* __restrict__ y, float* __restrict__ c,
                                                                  const float* __restrict__ e,
                                                                  const float* __restrict__ l,
                                                                  const float* __restrict__ u, TileFlush g,
                                                                  BatchMap lmap, BatchMap umap, int64_t nx,
                                                                  int64_t ny) {
  constexpr int H = WT / 2;               // tiles per wave per direction
  constexpr int ROWS = WT * TS;           // panel rows (A) / columns (B)
  constexpr int BPITCH = ROWS + 4;        // LDS pitch of the B panel rows (j fastest)
  constexpr int NV = ROWS * TS / 4 / 256; // float4 per thread per panel
  __shared__ __align__(16) float As[ROWS * AP];
  __shared__ __align__(16) float Bs[TS * BPITCH];

  const GridIds id = grid_ids(nx, ny);
  const int64_t b = id.b;
  const int64_t I0 = id.y * WT;
  int64_t jt_lo = g.S1 - (I0 + WT - 1);
  if (jt_lo < 0) jt_lo = 0;
  const int64_t J0 = (jt_lo / WT + id.x) * WT;
  if (J0 >= g.nt || I0 + J0 >= g.S_end || I0 + J0 + 2 * WT - 2 < g.S1) return;

  // workgroup-wide k ranges; nothing to do -> no memory touched
  int64_t lo0 = INT64_MAX, hi0 = 0, lo1 = INT64_MAX, hi1 = 0;
  for (int a = 0; a < WT; ++a)
    for (int d = 0; d < WT; ++d) {
      const int64_t I = I0 + a, J = J0 + d;
      if (!is_target(g, I, J)) continue;
      int64_t lo, hi;
      tile_range(g, 0, I, J, lo, hi);
      if (lo < hi) {
        lo0 = lo < lo0 ? lo : lo0;
        hi0 = hi > hi0 ? hi : hi0;
      }
      tile_range(g, 1, I, J, lo, hi);
      if (lo < hi) {
        lo1 = lo < lo1 ? lo : lo1;
        hi1 = hi > hi1 ? hi : hi1;
      }
    }
  if (lo0 >= hi0 && lo1 >= hi1) return;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hh = lane >> 5;
  const int wi = (wave >> 1) * H, wj = (wave & 1) * H;  // wave's first tile, relative to (I0, J0)
  const int64_t mat = b * g.m * g.n;
  const float* lb = l + lmap.offset(b);
  const float* ub = u + umap.offset(b);

  // per-tile k ranges of this wave (uniform)
  int64_t tlo[2][H][H], thi[2][H][H];
  bool tgt[H][H];
#pragma unroll
  for (int a = 0; a < H; ++a)
#pragma unroll
    for (int d = 0; d < H; ++d) {
      const int64_t I = I0 + wi + a, J = J0 + wj + d;
      tgt[a][d] = is_target(g, I, J);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        tile_range(g, p, I, J, tlo[p][a][d], thi[p][a][d]);
        if (!tgt[a][d]) thi[p][a][d] = tlo[p][a][d];
      }
    }

  floatx16 acc[H][H];
#pragma unroll
  for (int a = 0; a < H; ++a)
#pragma unroll
    for (int d = 0; d < H; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][d][r] = 0.f;

  float4 ra[NV], rb[NV];

#pragma unroll
  for (int phase = 0; phase < 2; ++phase) {
    const int64_t t_lo = phase == 0 ? lo0 : lo1, t_hi = phase == 0 ? hi0 : hi1;
    // A source: L (phase 0) or C (phase 1), rows of the WG, row-major with k fastest
    const float* abase = phase == 0 ? lb : c + mat;
    const int64_t alda = phase == 0 ? g.m : g.n;   // row stride of A
    const int64_t akmax = phase == 0 ? g.m : g.n;  // k extent of A
    // B source: E (phase 0) or U (phase 1), row-major with j fastest
    const float* bbase = phase == 0 ? e + mat : ub;
    const int64_t bkmax = phase == 0 ? g.m : g.n;  // k extent of B

    auto stage = [&](int64_t t) {
      const int64_t k0 = t * TS;
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int f = tid + 256 * q;
        // A: row r, k = 4 kq .. 4 kq + 3
        {
          const int r = f / (TS / 4), kq = f % (TS / 4);
          const int64_t i = I0 * TS + r, k = k0 + 4 * kq;
          const int64_t ti = i >> 5;
          const bool ok = i < g.m && (phase == 0 ? t < ti : (ti + t >= g.S0 && ti + t < g.S1));
          const float* src = abase + i * alda + k;
          float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
          if (VEC) {
            if (ok && k < akmax) v = *reinterpret_cast<const float4*>(src);
          } else if (ok) {
            v.x = k < akmax ? src[0] : 0.f;
            v.y = k + 1 < akmax ? src[1] : 0.f;
            v.z = k + 2 < akmax ? src[2] : 0.f;
            v.w = k + 3 < akmax ? src[3] : 0.f;
          }
          ra[q] = v;
        }
        // B: row kk, j = 4 cq .. 4 cq + 3 (one tile column per 8 float4)
        {
          const int kk = f / (ROWS / 4), cq = f % (ROWS / 4);
          const int64_t k = k0 + kk, j = J0 * TS + 4 * cq;
          const int64_t tj = j >> 5;
          const bool ok = k < bkmax && (phase == 0 ? (t + tj >= g.S0 && t + tj < g.S1) : t < tj);
          const float* src = bbase + k * g.n + j;
          float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
          if (VEC) {
            if (ok && j < g.n) v = *reinterpret_cast<const float4*>(src);
          } else if (ok) {
            v.x = j < g.n ? src[0] : 0.f;
            v.y = j + 1 < g.n ? src[1] : 0.f;
            v.z = j + 2 < g.n ? src[2] : 0.f;
            v.w = j + 3 < g.n ? src[3] : 0.f;
          }
          rb[q] = v;
        }
      }
    };

    if (t_lo < t_hi) stage(t_lo);
    for (int64_t t = t_lo; t < t_hi; ++t) {
      __syncthreads();
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int f = tid + 256 * q;
        const int r = f / (TS / 4), kq = f % (TS / 4);
        *reinterpret_cast<float4*>(&As[r * AP + 4 * kq]) = ra[q];
        const int kk = f / (ROWS / 4), cq = f % (ROWS / 4);
        *reinterpret_cast<float4*>(&Bs[kk * BPITCH + 4 * cq]) = rb[q];
      }
      __syncthreads();
      if (t + 1 < t_hi) stage(t + 1);

      bool ok[H][H];
      bool any = false;
#pragma unroll
      for (int a = 0; a < H; ++a)
#pragma unroll
        for (int d = 0; d < H; ++d) {
          ok[a][d] = t >= tlo[phase][a][d] && t < thi[phase][a][d];
          any |= ok[a][d];
        }
      if (!any) continue;
      float4 af[H][4];
#pragma unroll
      for (int a = 0; a < H; ++a) {
        const float* src = &As[((wi + a) * TS + li) * AP + 16 * hh];
#pragma unroll
        for (int v = 0; v < 4; ++v) af[a][v] = *reinterpret_cast<const float4*>(src + 4 * v);
      }
      const float* bsrc = &Bs[(16 * hh) * BPITCH + wj * TS + li];
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        float bf[H];
#pragma unroll
        for (int d = 0; d < H; ++d) bf[d] = bsrc[s * BPITCH + d * TS];
#pragma unroll
        for (int a = 0; a < H; ++a)
#pragma unroll
          for (int d = 0; d < H; ++d)
            if (ok[a][d]) acc[a][d] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[a][s >> 2][s & 3], bf[d], acc[a][d], 0,
                                                                           0, 0);
      }
    }

    // epilogue of the phase: C += D after the down products, Y += D + R after the right ones
#pragma unroll
    for (int a = 0; a < H; ++a)
#pragma unroll
      for (int d = 0; d < H; ++d) {
        const bool has = phase == 0 ? tlo[0][a][d] < thi[0][a][d]
                                    : (tlo[0][a][d] < thi[0][a][d] || tlo[1][a][d] < thi[1][a][d]);
        if (!has) continue;
        const int64_t I = I0 + wi + a, J = J0 + wj + d;
        float* dst = (phase == 0 ? c : y) + mat;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t i = I * TS + 8 * (r >> 2) + 4 * hh + (r & 3), j = J * TS + li;
          if (i < g.m && j < g.n) {
            const int64_t off = i * g.n + j;
            dst[off] = dst[off] + acc[a][d][r];
          }
        }
      }
  }
}

template <int WT>
int launch(float* y, float* c, const float* e, const float* l, const float* u, const TileFlush& g,
           const BatchMap& lmap, const BatchMap& umap, int64_t B, hipStream_t stream) {
  // block rows with targets, and the widest block-column range over them
  const int64_t rows_hi = g.S_end < g.mt ? g.S_end : g.mt;
  const int64_t nby = cdiv(rows_hi, WT);
  int64_t nbx = 0;
  for (int64_t by = 0; by < nby; ++by) {
    const int64_t I0 = by * WT;
    int64_t jt_lo = g.S1 - (I0 + WT - 1);
    if (jt_lo < 0) jt_lo = 0;
    int64_t jt_hi = g.S_end - 1 - I0;  // inclusive
    if (jt_hi > g.nt - 1) jt_hi = g.nt - 1;
    if (jt_hi < jt_lo) continue;
    const int64_t cnt = jt_hi / WT - jt_lo / WT + 1;
    if (cnt > nbx) nbx = cnt;
  }
  if (nbx == 0) return 0;
  Grid3 gr = make_grid(nbx, nby, B);
  const bool vec = g.m % 4 == 0 && g.n % 4 == 0;
  if (vec)
    hipLaunchKernelGGL((flush_tiles_mfma_kernel<WT, true>), gr.grid, dim3(256), 0, stream, y, c, e, l, u, g, lmap,
                       umap, gr.nx, gr.ny);
  else
    hipLaunchKernelGGL((flush_tiles_mfma_kernel<WT, false>), gr.grid, dim3(256), 0, stream, y, c, e, l, u, g, lmap,
                       umap, gr.nx, gr.ny);
  return (int)hipGetLastError();
}

}  // namespace

// Flush of tile stages [S0, S1) into [S1, S_end) on MFMA; 4 x 4 tiles per workgroup for wide bands
// of sources (outer flushes), 2 x 2 for single-stage bands.
int gptq2d_flush_tiles_mfma(float* y, float* c, const float* e, const float* l, const float* u, int64_t m, int64_t n,
                            int64_t S0, int64_t S1, int64_t S_end, const BatchMap& lmap, const BatchMap& umap,
                            int64_t B, hipStream_t stream) {
  TileFlush g{m, n, cdiv(m, TS), cdiv(n, TS), S0, S1, S_end};
  if (S1 - S0 >= 4) return launch<4>(y, c, e, l, u, g, lmap, umap, B, stream);
  return launch<2>(y, c, e, l, u, g, lmap, umap, B, stream);
}
