// Cross-tile flush of the fused sweep on MFMA: fp32 (v_mfma_f32_32x32x2_f32) and fp64
// (v_mfma_f64_16x16x4_f64, the same design with 2 x 2 such blocks per 32 x 32 tile).
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
// are loaded one k-tile ahead straight into LDS (buffer loads with the LDS destination bit, no
// register staging), double-buffered, one barrier per k-tile.  Staging loads are masked to
// exactly the entries a product may read: L strictly below, U strictly above its diagonal tiles,
// E and C on the band, nothing outside the matrix -- so a tile whose own range does not contain
// the k-tile multiplies zeros, and a wave runs its full MFMA block on every k-tile where any of
// its tiles is active (the union adds WT - 1 k-tiles per phase to a tile's range).  Tiles that
// receive nothing are not read or written.
//
// Operand layout, fp32 (lane l, i = l % 32, h = l / 32): A(i, kslot = h), B(kslot = h, j = i); the 16
// accumulators hold D(8 (r / 4) + 4 h + r % 4, i).  The k carried by slot h in MFMA s is 16 h + s
// for both operands, so 16 MFMAs cover the 32-deep k-tile.  fp64 (lane l, q = l % 16, h = l / 16), per
// 16 x 16 block: A(q, kslot = h), B(kslot = h, q); accumulator element r holds D(h + 4 r, q); the k of
// slot h in MFMA s is 8 h + s, so 8 MFMAs per block cover the k-tile.
//
// Reference counterparts (IST-DASLab/GPTQ-2D, gptq_2d.py): _flush_down_kernel :766-932 and
// _flush_right_kernel :936-1087 (fp32 `tl.dot` with input_precision="ieee"); one kernel here, with
// one read-modify-write of Y and C per target tile.
//
// LDS layouts are described at FlushLds: a lane reads its A values for one k-tile as four 128-bit
// reads, its B values as 32-bit reads (one per MFMA, paired by the compiler); the next group's
// fragments are read while the current group's MFMAs issue.
#include "common.h"
#include "lds_dma.h"

#include <type_traits>

namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef double doublex4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int TS = 32;      // tile edge (fp32: one MFMA block; fp64: 2 x 2 blocks)

// Accumulators of a wave's H x H tiles: one 32 x 32 fp32 block each, or 2 x 2 16 x 16 fp64 blocks.
template <typename T, int H>
struct AccOf {
  using type = floatx16[H][H];
};
template <int H>
struct AccOf<double, H> {
  using type = doublex4[H][H][2][2];
};

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

// The launch geometry in 32 bits for the kernel's work-item arithmetic (tile counts and stages stay
// below 2^15): the scalar unit compares 32-bit values itself, while 64-bit signed compares go
// through the vector unit and back -- a per-workgroup walk over the row blocks in 64 bits cost
// microseconds beside the MFMA waves of other workgroups.
struct TileGeo32 {
  int mt, nt, S0, S1, S_end;
};

__device__ __forceinline__ bool is_target(const TileGeo32& g, int I, int J) {
  return I < g.mt && J < g.nt && I + J >= g.S1 && I + J < g.S_end;
}

__device__ __forceinline__ void tile_range(const TileGeo32& g, int phase, int I, int J, int& lo, int& hi) {
  const int a = phase == 0 ? J : I, b = phase == 0 ? I : J;
  lo = g.S0 - a > 0 ? g.S0 - a : 0;
  hi = g.S1 - a < b ? g.S1 - a : b;
}

// Workgroups of a launch are exactly the (row block, column block) pairs that can hold targets:
// row block `by` (tile rows WT by ..) spans the column blocks [first, last] below.  Launching no
// empty workgroups matters: the dispatcher hands workgroups to the XCDs and shader engines in
// turn, and a stride of empty ones leaves whole engines idle while others queue.
template <int WT, typename G, typename Int>
__host__ __device__ inline void row_block_span(const G& g, Int by, Int& first, Int& count) {
  const Int I0 = by * WT;
  Int jt_lo = (Int)g.S1 - (I0 + WT - 1);
  if (jt_lo < 0) jt_lo = 0;
  Int jt_hi = (Int)g.S_end - 1 - I0;  // inclusive
  if (jt_hi > (Int)g.nt - 1) jt_hi = (Int)g.nt - 1;
  // a tile with I, J >= S1 receives nothing (its down range needs J < S1, its right range I < S1)
  if (I0 >= (Int)g.S1 && jt_hi > (Int)g.S1 - 1) jt_hi = (Int)g.S1 - 1;
  first = jt_lo / WT;
  count = (I0 < (Int)g.mt && jt_hi >= jt_lo) ? jt_hi / WT - first + 1 : 0;
}

// Order of the work items.  Row blocks are grouped in bands of SR, and a band's items are numbered column
// block by column block (inside a column by row block), so that a run of 16 consecutive items -- which go
// to one XCD, see the kernel -- is about 4 row blocks x 4 column blocks: every L / C row panel and E / U
// column panel the run streams through its L2 serves four of its workgroups (a run along one row block
// shares its row panel 16 ways and no column panel).
constexpr int SR = 4;

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    v += lane >= d ? o : 0;
  }
  return v;
}

// The entry of the sequence of counts f(0), f(1), ..., f(n - 1) that holds position k, with k reduced by the
// counts before it; -1 when k lies past the end.  Each lane evaluates one count per pass of 64 (wave-uniform
// result).
template <typename F>
__device__ __forceinline__ int wave_locate(const F& f, int n, int& k) {
  const int lane = threadIdx.x & 63;
  for (int base = 0; base < n; base += 64) {
    const int cnt = base + lane < n ? f(base + lane) : 0;
    const int s = wave_scan(cnt);
    const int tot = __builtin_amdgcn_readfirstlane(__shfl(s, 63, 64));
    if (k < tot) {
      const unsigned long long hit = __ballot(s > k);  // lane 63 at least
      const int j = __builtin_amdgcn_readfirstlane(__builtin_ctzll(hit));
      k -= __builtin_amdgcn_readfirstlane(__shfl(s - cnt, j, 64));
      return base + j;
    }
    k -= tot;
  }
  return -1;
}

// Row block `by` and column block `bx` of work item `item` (false past the last item).  Wave-parallel: a few
// hundred cycles, where a serial walk over the row blocks cost 10-36 thousand per workgroup at 8192^2.
template <int WT>
__device__ __forceinline__ bool item_block(const TileGeo32& q, int item, int& by, int& bx) {
  const int nby = (q.mt + WT - 1) / WT, nbands = (nby + SR - 1) / SR;
  auto band_items = [&](int band) {
    int tot = 0;
#pragma unroll
    for (int i = 0; i < SR; ++i) {
      int first = 0, count = 0;
      if (band * SR + i < nby) row_block_span<WT>(q, band * SR + i, first, count);
      tot += count;
    }
    return tot;
  };
  int k = item;
  const int band = wave_locate(band_items, nbands, k);
  if (band < 0) return false;
  int f[SR], c[SR], lo = INT32_MAX, hi = 0;  // the band's spans [f, f + c); columns [lo, hi)
#pragma unroll
  for (int i = 0; i < SR; ++i) {
    f[i] = c[i] = 0;
    if (band * SR + i < nby) row_block_span<WT>(q, band * SR + i, f[i], c[i]);
    if (c[i] > 0) {
      lo = f[i] < lo ? f[i] : lo;
      hi = f[i] + c[i] > hi ? f[i] + c[i] : hi;
    }
  }
  auto column_items = [&](int x) {
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < SR; ++i) cnt += lo + x >= f[i] && lo + x < f[i] + c[i] ? 1 : 0;
    return cnt;
  };
  const int x = wave_locate(column_items, hi - lo, k);
  if (x < 0) return false;
  bx = lo + x;
#pragma unroll
  for (int i = 0; i < SR; ++i)
    if (bx >= f[i] && bx < f[i] + c[i]) {
      if (k == 0) {
        by = band * SR + i;
        return true;
      }
      --k;
    }
  return false;
}

// Panels in LDS, per k-tile (ROWS = 32 WT), both double-buffered:
//   A (ROWS x 32 k; k contiguous in memory): element f holds row f / 32 and k = QE (q ^ swizzle(row)) +
//     f % QE with q = (f % 32) / QE -- the 16-byte k-quads of QE elements XOR-swizzled by row, so that the
//     rows that lanes read together at one k-quad lie in different bank groups (fp32: quad_swizzle of
//     lds_dma.h over a row's 8 quads; fp64: row % 16 over its 16 quads, distinct for the 16 consecutive rows
//     that the 16 lanes of a 128-bit read's cycle take, which then cover all 64 banks);
//   B (32 k x ROWS columns; columns contiguous in memory): k-row k at k ROWS, plus BPAD elements per group
//     of BGRP, so that the k-rows that one half-wave reads together fall 32 banks apart (fp32: rows k and
//     k + 16; fp64: rows k and k + 8).
template <typename T, int WT>
struct FlushLds {
  static_assert(sizeof(T) == 4 || WT == 2, "the fp64 layout is for 2 x 2-tile workgroups");
  static constexpr int QE = 16 / (int)sizeof(T);  // elements per 16-byte quad
  static constexpr int ROWS = WT * TS;
  static constexpr int PANEL = ROWS * TS;
  static constexpr int BGRP = sizeof(T) == 4 ? 256 : 512;
  static constexpr int BPAD = sizeof(T) == 4 ? 512 / ROWS : 16;
  static constexpr int BSZ = PANEL + PANEL / BGRP * BPAD;
  T a[2][PANEL];
  T b[2][BSZ];
};

template <typename T>
__device__ __forceinline__ int panel_swizzle(int row) {
  if constexpr (sizeof(T) == 4)
    return quad_swizzle(row);
  else
    return row & 15;
}

// An LDS panel address as the float pointer that the LDS-direct loads take (they move dwords).
template <typename T>
__device__ __forceinline__ float* lds_dst(T* p) {
  return reinterpret_cast<float*>(p);
}

// Buffer resource over the elements [first, total) of a matrix stored from `base`: offsets count from
// element `first`, so that they stay small whatever the matrix size (extents capped below OOB).
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rebased_rsrc(const T* base, int64_t first, int64_t total) {
  // clamped with shifts and 32-bit compares (the scalar unit has no 64-bit ordered compare, and these are
  // evaluated once per k-tile in the MFMA loops): a negative extent -> 0, a longer one than cap -> cap
  const uint64_t rem = (uint64_t)(total - first);
  constexpr unsigned cap = OOB / (int)sizeof(T) - 64;  // < 2^29 floats / 2^28 doubles
  unsigned hi = (unsigned)(rem >> 32);
  const unsigned lo = (unsigned)rem;
  asm("" : "+s"(hi));  // opaque: otherwise the tests below are folded back into 64-bit compares
  const unsigned elems = (hi >> 31) ? 0u : (hi != 0 || lo > cap ? cap : lo);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base + first), (short)0, (int)(elems * sizeof(T)),
                                           0x00020000);
}

// One product phase (0: D = L E, 1: R = C U) of a workgroup, accumulated into acc.  a_mat / b_mat: the
// operand matrices (a_elems / b_elems elements): A is staged through a buffer resource based at the
// workgroup's first row, B through one based at each k-tile's first row and the workgroup's first
// column, so that every offset stays below 2^31 bytes for any matrix a tile row or a k-tile of which does.
// KR (the right product with U = P (x) Q given by its factors, fp32, nq % 16 == 0): B is staged from Q, each
// 16-row half of a k-tile through a resource based at its first row of Q, and every B value is multiplied by its
// P entry when the fragments are read -- the U entries of the explicit product, bit for bit.  A lane's fragment
// values share one P entry per k-tile: its column is fixed, and its k slot covers 16 aligned rows.
template <typename T, int WT, bool VEC, int PHASE, bool KR = false>
__device__ __forceinline__ void flush_phase(typename AccOf<T, WT / 2>::type& acc, FlushLds<T, WT>& sm,
                                            const T* a_mat, int64_t a_elems, const T* b_mat, int64_t b_elems,
                                            const TileFlush& g, int64_t I0, int64_t J0, int wi, int wj,
                                            int t_lo, int t_hi, const int (&tlo)[WT / 2][WT / 2],
                                            const int (&thi)[WT / 2][WT / 2], const KronU& kr = KronU{},
                                            float* pk_lds = nullptr) {
  using L = FlushLds<T, WT>;
  static_assert(sizeof(T) == 4 || VEC, "fp64 panels are staged 128 bits at a time");
  static_assert(!KR || (sizeof(T) == 4 && VEC && WT == 2 && PHASE == 1), "U from its Kronecker factors: fp32 "
                "right products of 2 x 2-tile workgroups staged 128 bits at a time");
  constexpr int H = WT / 2;
  constexpr int ROWS = L::ROWS;
  constexpr int QE = L::QE;
  constexpr int ES = (int)sizeof(T);
  constexpr int W = VEC ? QE : 1;         // elements per lane per load (a 16-byte quad, or one float)
  constexpr int DW = W * ES / 4;          // dwords per lane per load
  constexpr int PER = 64 * W;             // elements per wave load
  constexpr int NI = L::PANEL / PER / 4;  // loads per wave per panel and k-tile
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS bases in scalar registers
  const int kmax = (int)(PHASE == 0 ? g.m : g.n);  // k extent of both operands
  const int alda = (int)(PHASE == 0 ? g.m : g.n);  // row stride of A (L or C)
  const int gm = (int)g.m, gn = (int)g.n, s0 = (int)g.S0, s1 = (int)g.S1;  // < 2^20: 32-bit index math
  const __amdgpu_buffer_rsrc_t ra_src = rebased_rsrc(a_mat, I0 * TS * (int64_t)alda, a_elems);

  // per-lane staging geometry of load x: A row i (tile at, k offset akk), B column j (tile bt, k row
  // kb); loop-invariant, so kept in registers for the 128-bit path (NI = 4) and recomputed for the
  // 32-bit one
  struct Geo {
    int a_off, a_t, a_kk, b_off, b_t, b_kb;
    bool a_in, b_in;
  };
  auto geo = [&](int x) {
    Geo o;
    const int f = (wave + 4 * x) * PER + lane * W;
    const int row = f / TS;
    o.a_kk = QE * (((f % TS) / QE) ^ panel_swizzle<T>(row)) + f % QE;
    const int i = (int)I0 * TS + row;
    o.a_in = i < gm;
    o.a_t = i >> 5;
    o.a_off = ((o.a_in ? row * alda : 0) + o.a_kk) * ES;  // from the workgroup's first row
    o.b_kb = f / ROWS;
    const int j = (int)J0 * TS + f % ROWS;
    o.b_in = j < gn;
    o.b_t = j >> 5;
    if constexpr (KR) {  // row kb % 16 of the half k-tile's rows of Q, column j % nq of Q
      int jb, jq;
      kron_index(kr, j, jb, jq);
      o.b_off = ((o.b_kb & 15) * kr.nq + (o.b_in ? jq : 0)) * ES;
    } else {
      o.b_off = (o.b_kb * gn + (o.b_in ? f % ROWS : 0)) * ES;  // from the k-tile's first row, the first column
    }
    return o;
  };
  Geo pre[VEC ? NI : 1];
  if constexpr (VEC) {
#pragma unroll
    for (int x = 0; x < NI; ++x) pre[x] = geo(x);
  }

  // whether the workgroup's A rows and B columns are whole tiles inside the matrix (uniform)
  const int i0t = (int)I0, j0t = (int)J0;
  const bool full = (i0t + WT) * TS <= gm && (j0t + WT) * TS <= gn;

  // KR: (block of P, 16-row unit of Q) of the first half of the next k-tile to stage (issue takes the k-tiles in
  // order, each once; uniform), and the byte offset in a row of P of the block of the workgroup's column `lane`
  // (clamped: a column past the matrix has its B values masked to zero).  The P entries of a k-tile -- its two
  // halves' blocks times the workgroup's 64 columns -- are staged into pk_lds[buffer][half][column] with the
  // panels (waves 0 and 1, one LDS-direct load each): P never passes through registers, so the compiler's own
  // waits for vector loads do not hold up the MFMAs of the k-tile before
  constexpr int LQ = sizeof(T) == 4 ? 32 : 16;  // lanes of one k slot of the fragments below
  const int li = lane % LQ, hh = lane / LQ;
  int kub = 0, kur = 0, pofs = 0;
  if constexpr (KR) {
    kron_split(kr, (unsigned)(2 * t_lo), kub, kur);
    int pb, jq;
    kron_index(kr, j0t * TS + lane < gn - 1 ? j0t * TS + lane : gn - 1, pb, jq);
    pofs = pb * 4;
  }

  // loads of k-tile t into buffer buf, each masked to what a product may read (L strictly below its
  // diagonal tiles, C and E on the band, U strictly above its diagonal tiles, nothing outside)
  auto issue = [&](int t, int buf) {
    const int ts = (int)t, k0 = ts * TS;
    __amdgpu_buffer_rsrc_t rb_src, rb_hi;  // KR: the k-tile's first and second halves of rows
    int b1 = 0, r1 = 0;                      // KR: the second half's block of P and unit of Q
    if constexpr (KR) {
      b1 = kub, r1 = kur + 1;
      if (r1 == kr.d16) r1 = 0, ++b1;
      rb_src = rebased_rsrc(kr.q, (int64_t)kur * 16 * kr.nq, (int64_t)kr.nq * kr.nq);
      rb_hi = rebased_rsrc(kr.q, (int64_t)r1 * 16 * kr.nq, (int64_t)kr.nq * kr.nq);
    } else {
      rb_src = rb_hi = rebased_rsrc(b_mat, (int64_t)k0 * gn + J0 * TS, b_elems);
    }
    // KR, after the panels: the k-tile's P entries into pk_lds (wave h stages half h), then the next k-tile's
    // position
    auto stage_p = [&]() {
      if constexpr (KR) {
        if (wave < 2) {
          const int pb = wave ? b1 : kub;
          dma_load<1>(rebased_rsrc(kr.p, (int64_t)pb * kr.np, (int64_t)kr.np * kr.np),
                      &pk_lds[(buf * 2 + wave) * ROWS], pofs);
        }
        kub = b1, kur = r1 + 1;
        if (kur == kr.d16) kur = 0, ++kub;
      }
    };
    // the B resource of load x: its four k-rows lie in one half of the k-tile
    auto rb_of = [&](int x) { return KR && (wave + 4 * x) * PER / ROWS >= 16 ? rb_hi : rb_src; };
    // an interior k-tile, where no lane of the workgroup is masked (every row and column inside the matrix and
    // every A row / B column tile inside its band or triangle -- all k-tiles of a product but its first and
    // last few): the loads take their loop-invariant lane offsets with the k-tile's offset added in the
    // scalar field, no vector instruction.  Vector work between the MFMA bursts is what the k-step waits
    // for (every vector instruction waits for an issue slot beside the other waves' MFMAs): the masked
    // form's 20-odd per k-tile had cost more cycles than the 16 MFMAs.
    if constexpr (VEC) {
      const bool inner = PHASE == 0 ? ts < i0t && ts + j0t >= s0 && ts + j0t + WT - 1 < s1
                                    : ts < j0t && ts + i0t >= s0 && ts + i0t + WT - 1 < s1;
      if (full && inner && k0 + TS <= kmax) {
#pragma unroll
        for (int x = 0; x < NI; ++x) {
          const int f0 = (wave + 4 * x) * PER;
          dma_load_so<DW>(ra_src, lds_dst(&sm.a[buf][f0]), pre[x].a_off, k0 * ES);
          dma_load<DW>(rb_of(x), lds_dst(&sm.b[buf][f0 + f0 / L::BGRP * L::BPAD]), pre[x].b_off);
        }
        stage_p();
        return;
      }
    }
#pragma unroll
    for (int x = 0; x < NI; ++x) {
      const Geo o = VEC ? pre[x] : geo(x);
      const int f0 = (wave + 4 * x) * PER;
      const bool aband = PHASE == 0 ? ts < o.a_t : (o.a_t + ts >= s0 && o.a_t + ts < s1);
      const bool aok = o.a_in && aband && k0 + o.a_kk < kmax;
      dma_load<DW>(ra_src, lds_dst(&sm.a[buf][f0]), aok ? o.a_off + k0 * ES : OOB);
      const bool bband = PHASE == 0 ? (ts + o.b_t >= s0 && ts + o.b_t < s1) : ts < o.b_t;
      const bool bok = o.b_in && bband && k0 + o.b_kb < kmax;
      dma_load<DW>(rb_of(x), lds_dst(&sm.b[buf][f0 + f0 / L::BGRP * L::BPAD]), bok ? o.b_off : OOB);
    }
    stage_p();
  };

  // fragments.  fp32: A tile a, k-quad 4 hh + v of row (wi + a) 32 + li; B tile d, k = 16 hh + s, column
  // (wj + d) 32 + li -- the k of MFMA s is 16 hh + s for both operands.  fp64 (one tile per wave): A block a2,
  // k-quad 4 hh + v of row 32 wi + 16 a2 + li; B block d2, k = 8 hh + s, column 32 wj + 16 d2 + li -- the k of
  // MFMA s is 8 hh + s for both operands
  const int kh = (sizeof(T) == 4 ? 16 : 8) * hh;  // first k of the lane's slot
  const int a_base = (wi * TS + li) * TS;
  const int sw = panel_swizzle<T>(li);
  const int b_base = kh * ROWS + wj * TS + li + kh * ROWS / L::BGRP * L::BPAD;

  auto step = [&](int t, auto cur_c) {
    constexpr int cur = decltype(cur_c)::value;
    __syncthreads();  // buffer cur is complete; buffer 1 - cur is no longer read
    if (t + 1 < t_hi) issue(t + 1, 1 - cur);
    // a wave skips a k-tile on which none of its tiles is active; otherwise it runs the full MFMA
    // block -- the staging masks have zeroed the operands of any tile outside its own range, so
    // the inactive tiles of a partial step accumulate exact zeros
    const int ts = t;
    int any = 0;  // wave-uniform; an int so that it stays in scalar registers
#pragma unroll
    for (int a = 0; a < H; ++a)
#pragma unroll
      for (int d = 0; d < H; ++d) any |= ts >= tlo[a][d] && ts < thi[a][d] ? 1 : 0;
    if constexpr (sizeof(T) == 8) {
      if (any) {
        const double* as = &sm.a[cur][a_base];
        const double* bs = &sm.b[cur][b_base];
        double2 fa[2][2];     // [slot][a2]: k-quad v, i.e. k = 8 hh + 2 v + (0, 1)
        double fb[2][2][2];   // [slot][d2][s2]: k = 8 hh + 2 v + s2
        auto frag = [&](int v, int slot) {
#pragma unroll
          for (int a2 = 0; a2 < 2; ++a2)
            fa[slot][a2] = *reinterpret_cast<const double2*>(as + a2 * 16 * TS + 2 * ((4 * hh + v) ^ sw));
#pragma unroll
          for (int d2 = 0; d2 < 2; ++d2)
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) fb[slot][d2][s2] = bs[16 * d2 + (2 * v + s2) * ROWS];
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
              for (int d2 = 0; d2 < 2; ++d2)
                acc[0][0][a2][d2] = __builtin_amdgcn_mfma_f64_16x16x4f64(fa[v & 1][a2][s2], fb[v & 1][d2][s2],
                                                                          acc[0][0][a2][d2], 0, 0, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    } else if (any) {
      const float* as = &sm.a[cur][a_base];
      const float* bs = &sm.b[cur][b_base];
      const float pkc = KR ? pk_lds[(cur * 2 + hh) * ROWS + wj * TS + li] : 0.f;  // KR: the lane's P entry
      float4 fa[2][H];
      float fb[2][H][4];
      auto frag = [&](int v, int slot) {
#pragma unroll
        for (int a = 0; a < H; ++a)
          fa[slot][a] = *reinterpret_cast<const float4*>(as + a * TS * TS + 4 * ((4 * hh + v) ^ sw));
#pragma unroll
        for (int d = 0; d < H; ++d)
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) {
            const int s = 4 * v + s2;
            fb[slot][d][s2] = bs[d * TS + s * ROWS + s * ROWS / L::BGRP * L::BPAD];
            if constexpr (KR) fb[slot][d][s2] *= pkc;
          }
      };
      frag(0, 0);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (v < 3) frag(v + 1, (v + 1) & 1);
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
          for (int a = 0; a < H; ++a)
#pragma unroll
            for (int d = 0; d < H; ++d)
              acc[a][d] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[v & 1][a][s2], fb[v & 1][d][s2], acc[a][d], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_dma();  // this wave's loads of k-tile t + 1 have landed before the next barrier
  };

  if (t_lo >= t_hi) return;
  __syncthreads();  // the previous phase's last reads of both buffers are done
  issue(t_lo, 0);
  wait_dma();
  for (int t = t_lo; t < t_hi; t += 2) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 < t_hi) step(t + 1, std::integral_constant<int, 1>{});
  }
}

template <typename T, int WT, bool VEC, bool KR = false>
__global__ __launch_bounds__(256, 2) void flush_tiles_mfma_kernel(T* __restrict__ y, T* __restrict__ c,
                                                                  const T* __restrict__ e, const T* __restrict__ l,
                                                                  const T* __restrict__ u, TileFlush g,
                                                                  BatchMap lmap, BatchMap umap, int64_t b0,
                                                                  KronU kr) {
  constexpr int H = WT / 2;        // tiles per wave per direction
  __shared__ __align__(16) FlushLds<T, WT> sm;
  __shared__ float pk_lds[KR ? 2 * 2 * 2 * TS : 1];  // KR: the P entries of each buffer's k-tile (flush_phase)

  // XCD-aware order: the hardware deals workgroup w to XCD w % 8; runs of XG consecutive work items
  // (about SR x SR neighbouring blocks, item_block) go to one XCD and its L2, and the XCDs take turns
  // run by run, so that all of them see the same mix of item sizes
  constexpr int XG = 16;
  const int nwg = (int)gridDim.x, w = (int)blockIdx.x;
  const int full = nwg / (8 * XG) * (8 * XG);
  int item = w;
  if (w < full) {
    const int within = w % (8 * XG);
    item = w - within + (within % 8) * XG + within / 8;
  }
  const int64_t b = b0 + blockIdx.y;
  const TileGeo32 q{(int)g.mt, (int)g.nt, (int)g.S0, (int)g.S1, (int)g.S_end};
  int by = 0, bx = 0;
  if (!item_block<WT>(q, item, by, bx)) return;
  const int I0 = by * WT;
  const int J0 = bx * WT;
  if (J0 >= q.nt || I0 + J0 >= q.S_end || I0 + J0 + 2 * WT - 2 < q.S1) return;

  // workgroup-wide k ranges; nothing to do -> no memory touched
  int lo0 = INT32_MAX, hi0 = 0, lo1 = INT32_MAX, hi1 = 0;
  for (int a = 0; a < WT; ++a)
    for (int d = 0; d < WT; ++d) {
      const int I = I0 + a, J = J0 + d;
      if (!is_target(q, I, J)) continue;
      int lo, hi;
      tile_range(q, 0, I, J, lo, hi);
      if (lo < hi) {
        lo0 = lo < lo0 ? lo : lo0;
        hi0 = hi > hi0 ? hi : hi0;
      }
      tile_range(q, 1, I, J, lo, hi);
      if (lo < hi) {
        lo1 = lo < lo1 ? lo : lo1;
        hi1 = hi > hi1 ? hi : hi1;
      }
    }
  if (lo0 >= hi0 && lo1 >= hi1) return;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps the tile masks scalar
  constexpr int LQ = sizeof(T) == 4 ? 32 : 16;  // lanes of one accumulator row group
  const int li = lane % LQ, hh = lane / LQ;
  const int wi = (wave >> 1) * H, wj = (wave & 1) * H;  // wave's first tile, relative to (I0, J0)
  const int64_t mat = b * g.m * g.n;

  // per-tile k ranges of this wave (uniform); an empty range for tiles that are not targets
  int tlo[2][H][H], thi[2][H][H];
#pragma unroll
  for (int a = 0; a < H; ++a)
#pragma unroll
    for (int d = 0; d < H; ++d) {
      const int I = I0 + wi + a, J = J0 + wj + d;
      const bool tgt = is_target(q, I, J);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        int lo, hi;
        tile_range(q, p, I, J, lo, hi);
        tlo[p][a][d] = lo;
        thi[p][a][d] = tgt ? hi : lo;
      }
    }

  typename AccOf<T, H>::type acc;
#pragma unroll
  for (int a = 0; a < H; ++a)
#pragma unroll
    for (int d = 0; d < H; ++d) {
      if constexpr (sizeof(T) == 8) {
#pragma unroll
        for (int x = 0; x < 16; ++x) acc[a][d][x >> 3][(x >> 2) & 1][x & 3] = 0.;
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[a][d][r] = 0.f;
      }
    }

  // phase 0: D = L E, then C += D; phase 1: R = C U on top of D, then Y += D + R
  const T* lm = l + lmap.offset(b);
  const T* um = KR ? nullptr : u + umap.offset(b);
  flush_phase<T, WT, VEC, 0>(acc, sm, lm, g.m * g.m, e + mat, g.m * g.n, g, I0, J0, wi, wj, lo0, hi0, tlo[0], thi[0]);
#pragma unroll
  for (int ph = 0; ph < 2; ++ph) {
    if (ph == 1)
      flush_phase<T, WT, VEC, 1, KR>(acc, sm, c + mat, g.m * g.n, um, g.n * g.n, g, I0, J0, wi, wj, lo1, hi1, tlo[1],
                                     thi[1], kr, pk_lds);
    // epilogue of the phase: C += D after the down products, Y += D + R after the right ones
#pragma unroll
    for (int a = 0; a < H; ++a)
#pragma unroll
      for (int d = 0; d < H; ++d) {
        const bool has = ph == 0 ? tlo[0][a][d] < thi[0][a][d]
                                 : (tlo[0][a][d] < thi[0][a][d] || tlo[1][a][d] < thi[1][a][d]);
        if (!has) continue;
        const int64_t I = I0 + wi + a, J = J0 + wj + d;
        // the target tile's rows from a resource based at its first row (offsets below 2^31 bytes)
        const __amdgpu_buffer_rsrc_t rd = rebased_rsrc(ph == 0 ? c + mat : y + mat, I * TS * g.n, g.m * g.n);
        // all 16 reads in flight before the first write; masked lanes address past the matrix
        int off[16];
        T cur[16];
        if constexpr (sizeof(T) == 8) {
          // element r of block (a2, d2) (x = 8 a2 + 4 d2 + r): row 16 a2 + hh + 4 r, column 16 d2 + li
#pragma unroll
          for (int x = 0; x < 16; ++x) {
            const int ri = 16 * (x >> 3) + hh + 4 * (x & 3), cj = 16 * ((x >> 2) & 1) + li;
            const int64_t i = I * TS + ri, j = J * TS + cj;
            off[x] = (i < g.m && j < g.n) ? (ri * (int)g.n + (int)j) * 8 : OOB;
            cur[x] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(rd, off[x], 0, 0));
          }
#pragma unroll
          for (int x = 0; x < 16; ++x)
            __builtin_amdgcn_raw_buffer_store_b64(
                __builtin_bit_cast(u32x2, cur[x] + acc[a][d][x >> 3][(x >> 2) & 1][x & 3]), rd, off[x], 0, 0);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int ri = 8 * (r >> 2) + 4 * hh + (r & 3);
            const int64_t i = I * TS + ri, j = J * TS + li;
            off[r] = (i < g.m && j < g.n) ? (ri * (int)g.n + (int)j) * 4 : OOB;
            cur[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rd, off[r], 0, 0));
          }
#pragma unroll
          for (int r = 0; r < 16; ++r)
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, cur[r] + acc[a][d][r]), rd, off[r], 0,
                                                  0);
        }
      }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

bool strides_mult(const BatchMap& bm, int q) {
  for (int d = 0; d < bm.nd; ++d)
    if (bm.stride[d] % q) return false;
  return true;
}

// Workgroups (target blocks of WT x WT tiles) of one launch, per batch entry.
template <int WT>
int64_t count_items(const TileFlush& g) {
  const int64_t rows_hi = g.S_end < g.mt ? g.S_end : g.mt;
  int64_t items = 0;
  for (int64_t by = 0; by * WT < rows_hi; ++by) {
    int64_t first, count;
    row_block_span<WT>(g, by, first, count);
    items += count;
  }
  return items;
}

template <typename T, int WT, bool VEC, bool KR = false>
int launch(T* y, T* c, const T* e, const T* l, const T* u, const TileFlush& g, const BatchMap& lmap,
           const BatchMap& umap, int64_t B, hipStream_t stream, const KronU& kr = KronU{}) {
  const int64_t items = count_items<WT>(g);
  if (items == 0 || B == 0) return 0;
  if (items > 0x7fffffff) return GPTQ2D_EUNSUPPORTED;
  for (int64_t b0 = 0; b0 < B; b0 += 65535) {
    const dim3 grid((unsigned)items, (unsigned)(B - b0 < 65535 ? B - b0 : 65535));
    hipLaunchKernelGGL((flush_tiles_mfma_kernel<T, WT, VEC, KR>), grid, dim3(256), 0, stream, y, c, e, l, u, g, lmap,
                       umap, b0, kr);
  }
  return (int)hipGetLastError();
}

// Matrices whose rows, batch strides and base addresses allow 128-bit staging (q elements per 16 bytes).
template <typename T>
bool quad_aligned(const T* y, const T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n,
                  const BatchMap& lmap, const BatchMap& umap) {
  constexpr int q = 16 / (int)sizeof(T);
  return m % q == 0 && n % q == 0 && aligned16(y) && aligned16(c) && aligned16(e) && aligned16(l) && aligned16(u) &&
         strides_mult(lmap, q) && strides_mult(umap, q);
}

}  // namespace

// Whether gptq2d_flush_tiles_mfma takes a flush of 32 x 32 coarse cells: its buffer resources are based at
// each panel, so 32-bit offsets hold for rows and k-tiles of up to 2^20 elements (m, n < 2^20); fp64 panels
// are staged 128 bits at a time only, so fp64 also needs m and n even and 16-byte aligned matrices.
template <typename T>
bool gptq2d_flush_tiles_mfma_fits(const T* y, const T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n,
                                  const BatchMap& lmap, const BatchMap& umap) {
  if (m >= ((int64_t)1 << 20) || n >= ((int64_t)1 << 20)) return false;
  return sizeof(T) == 4 || quad_aligned(y, c, e, l, u, m, n, lmap, umap);
}

// Flush of tile stages [S0, S1) into [S1, S_end) on MFMA.
template <typename T>
int gptq2d_flush_tiles_mfma(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t S0,
                            int64_t S1, int64_t S_end, const BatchMap& lmap, const BatchMap& umap, int64_t B,
                            hipStream_t stream) {
  if (!gptq2d_flush_tiles_mfma_fits(y, c, e, l, u, m, n, lmap, umap)) return GPTQ2D_EUNSUPPORTED;
  TileFlush g{m, n, cdiv(m, TS), cdiv(n, TS), S0, S1, S_end};
  // 2 x 2 tiles per workgroup (four resident per CU in fp32, two in fp64), whose fine grain evens out the
  // launch's last round over the chip.  4 x 4 fp32 items (two resident per CU; each k-tile's panels serve four
  // times the MFMAs) lose wherever measured, also in launches of many rounds: at 8192^2 99 against 96-98
  // TFLOP/s over a layer's flushes, at 8192 x 28672 (C5a, 6+ rounds) a sweep of 94.5 against 97.6 ms, the same
  // bits.  fp32 rows whose length is not a multiple of 4 (or matrices not 16-byte aligned) are staged 32 bits
  // at a time.
  const bool vec = quad_aligned(y, c, e, l, u, m, n, lmap, umap);
  if constexpr (sizeof(T) == 4) {
    if (!vec) return launch<T, 2, false>(y, c, e, l, u, g, lmap, umap, B, stream);
  }
  return launch<T, 2, true>(y, c, e, l, u, g, lmap, umap, B, stream);
}

// The same flush with U = P (x) Q read from its factors (fp32, one matrix): rows of y, c, e, l and of Q staged
// 128 bits at a time (m and n multiples of 4, 16-byte aligned matrices), m, n < 2^20.
int gptq2d_flush_tiles_mfma_kron(float* y, float* c, const float* e, const float* l, const KronU& kr, int64_t m,
                                 int64_t n, int64_t S0, int64_t S1, int64_t S_end, hipStream_t stream) {
  BatchMap none;
  make_batch_map(none, 0, nullptr, nullptr);
  if (m >= ((int64_t)1 << 20) || n >= ((int64_t)1 << 20) || n != (int64_t)kr.np * kr.nq ||
      !quad_aligned<float>(y, c, e, l, kr.q, m, n, none, none))
    return GPTQ2D_EUNSUPPORTED;
  TileFlush g{m, n, cdiv(m, TS), cdiv(n, TS), S0, S1, S_end};
  return launch<float, 2, true, true>(y, c, e, l, nullptr, g, none, none, 1, stream, kr);
}

#define GPTQ2D_FLUSH_TILES_INST(T)                                                                                  \
  template bool gptq2d_flush_tiles_mfma_fits<T>(const T*, const T*, const T*, const T*, const T*, int64_t, int64_t, \
                                                const BatchMap&, const BatchMap&);                                  \
  template int gptq2d_flush_tiles_mfma<T>(T*, T*, const T*, const T*, const T*, int64_t, int64_t, int64_t, int64_t, \
                                          int64_t, const BatchMap&, const BatchMap&, int64_t, hipStream_t);
GPTQ2D_FLUSH_TILES_INST(float)
GPTQ2D_FLUSH_TILES_INST(double)
