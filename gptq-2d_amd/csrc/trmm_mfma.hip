// Row-major fp32 products with one lower triangular operand, on MFMA (v_mfma_f32_32x32x2_f32): the
// levels of the LDL's triangular inverse (ldl.hip), where every product multiplies an inverted
// diagonal block, lower triangular with its upper triangle cleared to zeros.
//
//   D = alpha A B   for `batch` strided problems, A: M x K (row stride lda), B: K x N (ldb), D: M x N
//   tri = 1: B lower (B(k, j) = 0 for k < j)  -> block column J0.. needs only k >= J0
//   tri = 2: A lower (A(i, k) = 0 for k > i)  -> block row I0.. needs only k < I0 + 128
//
// A dense GEMM library multiplies the zero triangle too; skipping the k-tiles that only meet zeros
// halves the arithmetic of a triangular product.  The boundary k-tiles (where the triangle's edge
// crosses the block) are multiplied in full: the zeros stored there make the result exact.
//
// One workgroup per 128 x 128 block of D, four waves of 64 x 64 (2 x 2 MFMA tiles).  The K loop
// walks k-tiles of 32; both panels are loaded one k-tile ahead straight into LDS (buffer loads with
// the LDS destination bit), double-buffered, one barrier per k-tile -- the scheme of the sweep's
// outer flush (flush_mfma.hip), with the same LDS layouts: A (128 rows x 32 k) with its 16-byte
// k-quads XOR-swizzled by row (quad_swizzle, lds_dma.h), B (32 k-rows x 128 columns) padded by 4 floats per
// two k-rows.
// Loads past the matrices return zeros (buffer range checks), so ragged edges need no branches.
#include "common.h"
#include "lds_dma.h"
#include "linalg.h"

#include <type_traits>

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int TB = 128;  // block edge
constexpr int KT = 32;   // k-tile depth
constexpr int BPAD = 4;  // B panel: floats of padding per 256 (two k-rows of 128 columns)
constexpr int BSZ = TB * KT + TB * KT / 256 * BPAD;

struct TrmmLds {
  float a[2][TB * KT];
  float b[2][BSZ];
};

__global__ __launch_bounds__(256, 2) void tri_gemm_kernel(TriGemm g, int64_t nbn) {
  __shared__ __align__(16) TrmmLds sm;
  // blocks renumbered so that each XCD (own L2) runs a contiguous share: neighbouring blocks of a
  // block row share their A panels
  const int64_t nwg = gridDim.x, w = blockIdx.x;
  const int64_t base = nwg / 8, extra = nwg % 8, xcd = w % 8;
  const int64_t lin = xcd * base + (xcd < extra ? xcd : extra) + w / 8;
  int bi = (int)(lin / nbn);
  const int bj = (int)(lin % nbn);
  if (g.tri == 2) {
    // a block row's k range grows with its index: rows taken as 0, last, 1, last - 1, ... so that
    // every XCD's contiguous share mixes long and short rows
    const int nbm = (int)((g.M + TB - 1) / TB), q = bi;
    bi = (q & 1) ? nbm - 1 - (q >> 1) : (q >> 1);
  }
  const int I0 = bi * TB, J0 = bj * TB;
  const int M = (int)g.M, N = (int)g.N, K = (int)g.K;
  const int lda = (int)g.lda, ldb = (int)g.ldb, ldd = (int)g.ldd;
  const float* A = g.A + (int64_t)blockIdx.y * g.sa + (int64_t)blockIdx.z * g.sa2;
  const float* B = g.B + (int64_t)blockIdx.y * g.sb + (int64_t)blockIdx.z * g.sb2;
  float* D = g.D + (int64_t)blockIdx.y * g.sd + (int64_t)blockIdx.z * g.sd2;

  const int nkt = (K + KT - 1) / KT;
  int t_lo = 0, t_hi = nkt;
  if (g.tri == 1) t_lo = J0 / KT;
  if (g.tri == 2) t_hi = (I0 + TB + KT - 1) / KT < nkt ? (I0 + TB + KT - 1) / KT : nkt;

  const int tid = threadIdx.x, lane = tid & 63, li = lane & 31, hh = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // buffer resources based at the block's rows of A and, per k-tile, at the k-tile's rows of B, so that every
  // byte offset stays below 128 rows of lda (A) or 32 rows of ldb (B) floats at any operand size
  const int arows = M - I0 < TB ? M - I0 : TB;
  const __amdgpu_buffer_rsrc_t ra = matrix_rsrc(A + (int64_t)I0 * lda, (int64_t)(arows - 1) * lda + K);
  auto b_rsrc = [&](int k0) {
    const int krows = K - k0 < KT ? K - k0 : KT;
    return matrix_rsrc(B + (int64_t)k0 * ldb + J0, (int64_t)(krows - 1) * ldb + (N - J0));
  };

  // per-lane staging of the wave's four 128-bit loads per panel and k-tile: A row `arow`, k-quad
  // akq (swizzled); B k-row bk, columns bcol .. bcol + 3
  int aoff[4], akk[4], boff[4], bk[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int f = (wave + 4 * x) * 256 + 4 * lane;
    const int row = f >> 5, kq = ((f >> 2) & 7) ^ quad_swizzle(row);
    akk[x] = 4 * kq;
    aoff[x] = row < arows ? (row * lda + akk[x]) * 4 : OOB;
    bk[x] = f >> 7;
    const int col = f & (TB - 1);
    boff[x] = J0 + col < N ? (bk[x] * ldb + col) * 4 : OOB;
  }
  // a block whose rows and columns all lie inside D takes its interior k-tiles (every lane in range) with
  // the k offset in the loads' scalar field: no vector instruction beside the MFMA bursts
  const bool full = I0 + TB <= M && J0 + TB <= N;
  auto issue = [&](int t, int buf) {
    const int k0 = t * KT;
    const __amdgpu_buffer_rsrc_t rb = b_rsrc(k0);
    if (full && k0 + KT <= K) {
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int f0 = (wave + 4 * x) * 256;
        dma_load_so<4>(ra, &sm.a[buf][f0], aoff[x], k0 * 4);
        dma_load_so<4>(rb, &sm.b[buf][f0 + f0 / 256 * BPAD], boff[x], 0);
      }
      return;
    }
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int f0 = (wave + 4 * x) * 256;
      const bool aok = aoff[x] != OOB && k0 + akk[x] < K;
      dma_load<4>(ra, &sm.a[buf][f0], aok ? aoff[x] + k0 * 4 : OOB);
      const bool bok = boff[x] != OOB && k0 + bk[x] < K;
      dma_load<4>(rb, &sm.b[buf][f0 + f0 / 256 * BPAD], bok ? boff[x] : OOB);
    }
  };

  floatx16 acc[2][2];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[a][d][r] = 0.f;

  // fragments: A tile a, k-quad 4 hh + v of row 64 wy + 32 a + li; B tile d, k = 16 hh + s, column
  // 64 wx + 32 d + li -- the k of MFMA s is 16 hh + s for both operands
  const int wy = wave >> 1, wx = wave & 1;
  const int a_base = (64 * wy + li) * KT, sw = quad_swizzle(li);
  const int b_base = 16 * hh * TB + 64 * wx + li + 16 * hh * TB / 256 * BPAD;
  auto step = [&](int t, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    __syncthreads();  // buffer cur is complete; buffer 1 - cur is no longer read
    if (t + 1 < t_hi) issue(t + 1, 1 - cur);
    const float* as = &sm.a[cur][a_base];
    const float* bs = &sm.b[cur][b_base];
    float4 fa[2][2];
    float fb[2][2][4];
    auto frag = [&](int v, int slot) {
#pragma unroll
      for (int a = 0; a < 2; ++a)
        fa[slot][a] = *reinterpret_cast<const float4*>(as + a * 32 * KT + 4 * ((4 * hh + v) ^ sw));
#pragma unroll
      for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) {
          const int s = 4 * v + s2;
          fb[slot][d][s2] = bs[32 * d + s * TB + s * TB / 256 * BPAD];
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
    wait_dma();  // this wave's loads of k-tile t + 1 have landed before the next barrier
  };
  if (t_lo < t_hi) {
    issue(t_lo, 0);
    wait_dma();
    for (int t = t_lo; t < t_hi; t += 2) {
      step(t, std::integral_constant<int, 0>{});
      if (t + 1 < t_hi) step(t + 1, std::integral_constant<int, 1>{});
    }
  }
  const float alpha = g.alpha;
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int j = J0 + 64 * wx + 32 * d + li;
      if (j >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int i = I0 + 64 * wy + 32 * a + 8 * (r >> 2) + 4 * hh + (r & 3);
        if (i < M) D[(int64_t)i * ldd + j] = alpha * acc[a][d][r];
      }
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

int gptq2d_tri_gemm_f32(const TriGemm& g, hipStream_t stream) {
  if (g.M < 0 || g.N < 0 || g.K < 0 || g.batch < 0 || g.tri < 0 || g.tri > 2 || g.batch2 < 0 || g.batch2 > 65535)
    return GPTQ2D_EINVAL;
  const unsigned nz = g.batch2 > 1 ? (unsigned)g.batch2 : 1u;
  if (g.M == 0 || g.N == 0 || g.batch == 0) return 0;
  if ((g.sa2 % 4 || g.sb2 % 4) && nz > 1) return GPTQ2D_EUNSUPPORTED;
  // 128-bit staging: rows and the block offsets of every operand on 16-byte boundaries
  if (g.K % 4 || g.N % 4 || g.lda % 4 || g.ldb % 4 || g.sa % 4 || g.sb % 4 || !aligned16(g.A) || !aligned16(g.B))
    return GPTQ2D_EUNSUPPORTED;
  // 32-bit byte offsets inside a block's 128 rows of A (plus K) and a k-tile's 32 rows of B (plus N)
  const int64_t lim = (int64_t)1 << 29;
  if (TB * g.lda + g.K >= lim || KT * g.ldb + g.N >= lim || g.M >= lim || g.N >= lim || g.K >= lim || g.K == 0)
    return GPTQ2D_EUNSUPPORTED;
  const int64_t nbm = (g.M + TB - 1) / TB, nbn = (g.N + TB - 1) / TB;
  if (nbm * nbn > 0x7fffffff) return GPTQ2D_EUNSUPPORTED;
  for (int64_t b0 = 0; b0 < g.batch; b0 += 65535) {
    TriGemm h = g;
    h.A += b0 * g.sa;
    h.B += b0 * g.sb;
    h.D += b0 * g.sd;
    const unsigned nb = (unsigned)(g.batch - b0 < 65535 ? g.batch - b0 : 65535);
    hipLaunchKernelGGL(tri_gemm_kernel, dim3((unsigned)(nbm * nbn), nb, nz), dim3(256), 0, stream, h, nbn);
    const int rc = (int)hipGetLastError();
    if (rc) return rc;
  }
  return 0;
}
