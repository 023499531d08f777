// Trellis (QTIP bitshift) quantizer: the Viterbi search of the closest trellis path, with
// tail-biting, in one launch per call.
//
// A state is an L-bit window of a bitstream; each step shifts KV = K*V new bits in, so the
// predecessors of state s are h * G + (s >> KV), h < 2^KV, with G = 2^(L-KV), and state s emits
// table[s, 0..V).  With cost_0(s) = d(s, x_0) and cost_t(s) = best_{t-1}(s >> KV) + d(s, x_t), where
// best_t(j) = min_h cost_t(h G + j) and d(s, x) = (table[s,0] - x0)^2 (+ (table[s,1] - x1)^2), the
// closest path ends in the first argmin of cost_{last}, and each earlier state is the first
// argmin over h of cost_{t-1}(h G + (state_t >> KV)).
//
// One workgroup (1024 threads) per one or two sequences runs every step of both tail-biting passes
// (two when 512 rows or more fill the chip and their minima fit in LDS: each table entry, read from
// L2 once per step, then serves both -- the table reads, not the arithmetic, bound the search): the
// group minima of the previous step sit in LDS (double-buffered, or read back from the history when
// 2 G values do not fit), each thread evaluates the 2^KV predecessors of its groups in order, and
// every step's minima are also stored in an HBM history [steps - 1][G] per sequence.  The final argmin is a
// block reduction; the walk back is done by one wave that recomputes the 2^KV candidate costs of the
// path's group at each step from the history -- the exact operations of the forward pass, so it picks
// the predecessor the search picked.  Tail-biting: pass 1 reads x rotated by half a sequence
// (through indices) and walks back only to the middle to fix the L - KV bits that the first and the
// last state share; pass 2 restricts the first state to (s >> KV) == overlap and the last to
// (s & (G - 1)) == overlap.
//
// Numerics as the reference: d0*d0 + d1*d1 then prev + that, no contraction into FMA (this file is
// compiled with -ffp-contract=off), ties to the first index.
//
// Reference: IST-DASLab/GPTQ-2D quantizer_trellis.py: _viterbi :82-115, _trellis_quantize_torch
// :118-143 (semantics), _viterbi_step/final/backtrack_kernel and _trellis_quantize_triton :146-341
// (the same search as 2 x (T/V + 1) launches per call).
#include "common.h"

#include <type_traits>

namespace {

constexpr int VT_THREADS = 1024;

template <typename T, int V>
__device__ __forceinline__ T local_cost(const T* __restrict__ table, int64_t s, T x0, T x1) {
  const T d0 = table[s * V] - x0;
  T c = d0 * d0;
  if constexpr (V == 2) {
    const T d1 = table[s * V + 1] - x1;
    c = c + d1 * d1;
  }
  return c;
}

// 16 bytes of a buffer at byte offset voff + soff (soff wave-uniform, in the scalar field).
__device__ __forceinline__ float4 table_quad(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  typedef float f4e __attribute__((ext_vector_type(4)));
  const f4e v = __builtin_bit_cast(f4e, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  return make_float4(v.x, v.y, v.z, v.w);
}

template <typename T>
__device__ __forceinline__ T inf_value() {
  return __builtin_huge_val();
}
template <>
__device__ __forceinline__ float inf_value<float>() {
  return __builtin_huge_valf();
}

// (value, index) that is smaller, ties to the smaller index.  As torch's argmin, a scan whose
// candidates are all +inf (every state masked) returns its first candidate: each scan takes its
// first candidate unconditionally and later ones only when strictly smaller.
template <typename T>
__device__ __forceinline__ void arg_better(T& v, int64_t& i, T v2, int64_t i2) {
  if (v2 < v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

template <typename T>
__device__ __forceinline__ T shfl_xor_t(T v, int mask) {
  return __shfl_xor(v, mask, 64);
}
__device__ __forceinline__ int64_t shfl_xor_t(int64_t v, int mask) {
  const int lo = __shfl_xor((int)(v & 0xffffffffll), mask, 64);
  const int hi = __shfl_xor((int)(v >> 32), mask, 64);
  return ((int64_t)hi << 32) | (unsigned int)lo;
}

template <typename T>
__device__ __forceinline__ void wave_argmin(T& v, int64_t& i) {
#pragma unroll
  for (int mask = 32; mask >= 1; mask >>= 1) {
    const T v2 = shfl_xor_t(v, mask);
    const int64_t i2 = shfl_xor_t(i, mask);
    arg_better(v, i, v2, i2);
  }
}

struct SearchGeom {
  int L, KV, steps;
  int64_t G;
  bool vec4;  // fp32, G % 4 == 0, KV >= 2, table and history on 16-byte boundaries
};

template <typename T, int V>
struct Sequence {
  const T* x;  // [steps * V]
  int steps;
  __device__ __forceinline__ void at(int t, int roll, T& x0, T& x1) const {
    const int tt = (t + roll) % steps;
    x0 = x[(int64_t)tt * V];
    x1 = V == 2 ? x[(int64_t)tt * V + 1] : T(0);
  }
};

// Final step of a forward pass: the first argmin over all states of cost_{last} (under the tail-biting masks),
// per sequence, into best_state[k]; the previous step's minima from LDS (prev_lds) or the history.
template <typename T, int V, int NS>
__device__ void final_argmin(const Sequence<T, V> (&seq)[NS], const T* __restrict__ table, T* const (&hist)[NS],
                             T* prev_lds, const SearchGeom& g, int roll, bool masked, const int64_t (&overlap)[NS],
                             int64_t* best_state, T* red_v, int64_t* red_i) {
  const int tid = threadIdx.x;
  const int64_t G = g.G;
  const T inf = inf_value<T>();
  const int last = g.steps - 1;
  const int64_t S = G << g.KV;
  const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    T x0, x1;
    seq[k].at(last, roll, x0, x1);
    T* pl = prev_lds ? prev_lds + k * 2 * G : nullptr;
    const T* prev = last == 0 ? nullptr : (pl ? pl + ((last - 1) & 1) * G : hist[k] + (int64_t)(last - 1) * G);
    T bv = inf;
    int64_t bi = INT64_MAX;
    for (int64_t s = tid; s < S; s += VT_THREADS) {
      T c = local_cost<T, V>(table, s, x0, x1);
      if (last == 0) {
        if (masked && (s >> g.KV) != overlap[k]) c = inf;
      } else {
        c = prev[s >> g.KV] + c;
      }
      if (masked && (s & (G - 1)) != overlap[k]) c = inf;
      if (c < bv || bi == INT64_MAX) {  // increasing s per thread: the first, then strictly smaller ones
        bv = c;
        bi = s;
      }
    }
    wave_argmin(bv, bi);
    if (lane == 0) {
      red_v[k * (VT_THREADS / 64) + wave] = bv;
      red_i[k * (VT_THREADS / 64) + wave] = bi;
    }
  }
  __syncthreads();
  if (tid < NS) {
    const int k = tid;
    T v = red_v[k * (VT_THREADS / 64)];
    int64_t i = red_i[k * (VT_THREADS / 64)];
    for (int w = 1; w < VT_THREADS / 64; ++w) arg_better(v, i, red_v[k * (VT_THREADS / 64) + w], red_i[k * (VT_THREADS / 64) + w]);
    best_state[k] = i & (S - 1);  // every state is a candidate, so i < S; the mask only keeps reads in bounds
  }
  __syncthreads();
}

// Forward pass of NS sequences in lockstep (the workgroup's): history_k[t][j] = best_t(j) of sequence
// k for t < steps - 1, and best_state[k] the first argmin of its cost_{last} under the masks.  Each
// table entry is loaded once per step for all NS sequences.  prev_lds: NS x 2 G values of LDS, or
// nullptr (then the previous step's minima are read back from the history).  Sequences with
// live[k] false are computed on a valid stand-in (their x pointer) but write nothing.
template <typename T, int V, int NS>
__device__ void forward_pass(const Sequence<T, V> (&seq)[NS], const bool (&live)[NS], const T* __restrict__ table,
                             T* const (&hist)[NS], T* prev_lds, const SearchGeom& g, int roll, bool masked,
                             const int64_t (&overlap)[NS], int64_t* best_state, T* red_v, int64_t* red_i) {
  const int tid = threadIdx.x;
  const int64_t G = g.G, H = (int64_t)1 << g.KV;
  const T inf = inf_value<T>();
  for (int t = 0; t + 1 < g.steps; ++t) {
    T x0[NS], x1[NS];
    const T* prev[NS];
    T* cur_lds[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      seq[k].at(t, roll, x0[k], x1[k]);
      T* pl = prev_lds ? prev_lds + k * 2 * G : nullptr;
      // at t = 0 a readable stand-in (its values are not used): the branch-free step below reads it
      prev[k] = t == 0 ? (pl ? pl : hist[k]) : (pl ? pl + ((t - 1) & 1) * G : hist[k] + (int64_t)(t - 1) * G);
      cur_lds[k] = pl ? pl + (t & 1) * G : nullptr;
    }
    // 32-bit state arithmetic (2^L <= 2^24 states)
    const int G32 = (int)G, H32 = (int)H, kv = g.KV;
    if constexpr (sizeof(T) == 4) {
      if (g.vec4) {
        // four consecutive groups j .. j + 3 per thread: for each h their states h G + j .. + 3 are
        // consecutive, so their table entries come in 128-bit loads (one per 4 V floats), and with
        // KV >= 2 they share the predecessor group s >> KV, whose minimum is read once per sequence;
        // the operations of each state evaluation are those of the loop below
        // the first step and the others as separate loops (no per-evaluation select on t == 0)
        // PL: the previous minima are in LDS (prev_lds), read and written through LDS-typed pointers --
        // through the generic ones the compiler emits flat accesses, whose waits also wait for the table's
        // loads in flight
        const __amdgpu_buffer_rsrc_t trs =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(table), (short)0, (int)((int64_t)(G << kv) * V * 4), 0x00020000);
        auto groups = [&](auto first_c, auto pl_c) {
        constexpr bool first = decltype(first_c)::value, PL = decltype(pl_c)::value;
        using lds_ct = const __attribute__((address_space(3))) T*;
        typedef float f4v __attribute__((ext_vector_type(4)));
        using lds_t4 = __attribute__((address_space(3))) f4v*;
        const T* prev_g[NS];
        lds_ct prev_l[NS];
#pragma unroll
        for (int k = 0; k < NS; ++k) {
          prev_g[k] = prev[k];
          prev_l[k] = PL ? (lds_ct)prev[k] : nullptr;
        }
        for (int j = 4 * tid; j < G32; j += 4 * VT_THREADS) {
          T best[NS][4];
#pragma unroll
          for (int k = 0; k < NS; ++k)
#pragma unroll
            for (int e = 0; e < 4; ++e) best[k][e] = inf;
          // the next h's table entries are loaded before this h's states are evaluated, so that each
          // load has a whole iteration to arrive (loaded and used in one iteration, every iteration
          // waited out the L2 latency)
          // through a buffer resource: this lane's byte offset fixed, step h's in the scalar field (no
          // 64-bit vector address arithmetic per load)
          const int tvo = j * V * 4, tstep = G32 * V * 4;
          float4 nxt[V];
#pragma unroll
          for (int q = 0; q < V; ++q) nxt[q] = table_quad(trs, tvo + 16 * q, 0);
#pragma unroll 2  // 4 or 8: 1.98-2.00 ms for a 512-sequence call, 2: 1.92 ms
          for (int h = 0; h < H32; ++h) {
            const int s = h * G32 + j;
            T tv[4 * V];
#pragma unroll
            for (int q = 0; q < V; ++q) {
              const float4 f = nxt[q];
              tv[4 * q] = f.x;
              tv[4 * q + 1] = f.y;
              tv[4 * q + 2] = f.z;
              tv[4 * q + 3] = f.w;
            }
            const int hn = h + 1 < H32 ? h + 1 : h;  // no branch: the last iteration reloads its own
#pragma unroll
            for (int q = 0; q < V; ++q) nxt[q] = table_quad(trs, tvo + 16 * q, hn * tstep);
            // issued here, not sunk to their use by the scheduler: one sequence per workgroup only (with two,
            // each h has twice the evaluations to cover the latency, and pinning the loads slowed it down)
            if constexpr (NS == 1) __builtin_amdgcn_sched_barrier(0);
            const int ps = s >> kv;
#pragma unroll
            for (int k = 0; k < NS; ++k) {
              const T pv = first ? T(0) : (PL ? prev_l[k][ps] : prev_g[k][ps]);
              const bool masked_out = first && masked && ps != overlap[k];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const T d0 = tv[V * e] - x0[k];
                T c = d0 * d0;
                if constexpr (V == 2) {
                  const T d1 = tv[V * e + 1] - x1[k];
                  c = c + d1 * d1;
                }
                if constexpr (first)
                  c = masked_out ? inf : c;
                else
                  c = pv + c;
                best[k][e] = fmin(c, best[k][e]);
              }
            }
          }
#pragma unroll
          for (int k = 0; k < NS; ++k) {
            const float4 b4 = make_float4(best[k][0], best[k][1], best[k][2], best[k][3]);
            if (live[k]) *reinterpret_cast<float4*>(hist[k] + (int64_t)t * G + j) = b4;
            if constexpr (PL)
              *(lds_t4)(cur_lds[k] + j) = f4v{b4.x, b4.y, b4.z, b4.w};
          }
        }
        };
        if (prev_lds) {
          if (t == 0)
            groups(std::true_type{}, std::true_type{});
          else
            groups(std::false_type{}, std::true_type{});
        } else {
          if (t == 0)
            groups(std::true_type{}, std::false_type{});
          else
            groups(std::false_type{}, std::false_type{});
        }
        __syncthreads();
        continue;
      }
    }
    for (int j = tid; j < G32; j += VT_THREADS) {
      T best[NS];
#pragma unroll
      for (int k = 0; k < NS; ++k) best[k] = inf;
      const bool first = t == 0;
#pragma unroll 16
      for (int h = 0; h < H32; ++h) {
        const int s = h * G32 + j;
        const T t0 = table[s * V];
        const T t1 = V == 2 ? table[s * V + 1] : T(0);
        const int ps = s >> kv;
#pragma unroll
        for (int k = 0; k < NS; ++k) {
          const T d0 = t0 - x0[k];
          T c = d0 * d0;
          if constexpr (V == 2) {
            const T d1 = t1 - x1[k];
            c = c + d1 * d1;
          }
          const T pv = prev[k][ps];
          c = first ? (masked && ps != overlap[k] ? inf : c) : pv + c;
          best[k] = fmin(c, best[k]);  // costs are never NaN: the same value as c < best ? c : best
        }
      }
#pragma unroll
      for (int k = 0; k < NS; ++k) {
        if (live[k]) hist[k][(int64_t)t * G + j] = best[k];
        if (cur_lds[k]) cur_lds[k][j] = best[k];
      }
    }
    __syncthreads();
  }
  final_argmin<T, V, NS>(seq, table, hist, prev_lds, g, roll, masked, overlap, best_state, red_v, red_i);
}

// ------------------------------------------------------------------------------------------------ few distinct rows
//
// Codes whose 2^L table rows take few distinct values -- HYB: 2^9 look-up rows times the sign of the first
// value; 1MAD: 908 values at L = 16 -- search from a per-step cost table instead of the table itself.  The table is
// given as E entries of W rows each, urows[E][W][V], and ridx[s] for s < 2^L / W: the entry whose row w is
// the row of state s + w 2^L / W (table[s + w 2^L / W] == urows[ridx[s]][w] bit for bit).  W = 2 pairs the
// states h G + j and (h + H / 2) G + j of a group (HYB: the same look-up row with both signs, 1024 ordered pairs);
// W = 1 is the plain distinct rows.  Each step first evaluates d(row, x_t) of every entry's rows (thread e,
// the same operations as every state evaluation of forward_pass), double-buffered in LDS; a state's
// evaluation is then that cost, read from LDS (one 8-byte read for the W = 2 states of an entry), plus the
// predecessor minimum and the running minimum.  The costs are the same values, so the search is the same.
// One sequence per workgroup; thread tid owns the four groups j = 4 tid .. 4 tid + 3 (G <= 4 VT_THREADS) and
// keeps the byte offsets of its (H / W) x 4 entries in the cost table in registers, two 16-bit offsets a
// register.
//
// The states' reads are random gathers: 32 lanes of 8 bytes (W = 2) or 64 lanes of 4 bytes (W = 1) meet the
// 64 four-byte banks, and the busiest bank sets the cycles of the read (3.4 deep on average for HYB's pairs
// against 1).  With copies == 2 each step's table is written twice, the second copy with its entries rotated
// in every row of banks (entry e of row r = e / NB at bank (e + r) mod NB, NB = 64 / W entries a row), and
// bit 16 of ridx[s] sends state s's reads to the second copy: a host-side choice per state that spreads each
// read's lanes over the banks (2.0 deep).  Either copy holds the same values.
constexpr int ROWS_MAX = 1024;

// the slot of entry e in the second copy: rotated by its row within its row of NB entries
template <int W>
__device__ __forceinline__ int second_slot(int e) {
  constexpr int NB = 64 / W;
  return (e & ~(NB - 1)) | ((e + e / NB) & (NB - 1));
}

template <int V, int H, int W, int PS>
__device__ void forward_rows(const Sequence<float, V>& sq, const float* xs, bool live, const float* __restrict__ table,
                             const float (&urow)[W][V], int E, int Ep, int copies, const int* __restrict__ ridx,
                             float* ctab, float* hist, float* prev_lds, const SearchGeom& g, int roll, bool masked,
                             int64_t overlap, int64_t* best_state, float* red_v, int64_t* red_i) {
  constexpr int HE = H / W;  // entries per group
  using lds_f = __attribute__((address_space(3))) float*;
  using lds_cf = const __attribute__((address_space(3))) float*;
  using lds_cb = const __attribute__((address_space(3))) char*;
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef float f4v __attribute__((ext_vector_type(4)));
  using lds_cf2 = const __attribute__((address_space(3))) f2v*;
  using lds_f4 = __attribute__((address_space(3))) f4v*;
  const int tid = threadIdx.x;
  const int G32 = (int)g.G, kv = g.KV;
  const float inf = __builtin_huge_valf();
  const int j = 4 * tid;
  const bool owner = j < G32;
  // the byte offsets of this thread's entries' costs in a buffer, loaded here (not held across the walks back):
  // entry ridx & 0xffff (clamped to the table), in the second copy where bit 16 is set and two are written
  const int cmask = copies - 1;
  auto slot_bytes = [&](int r) -> uint32_t {  // branch-free: a branch per entry costs scalar registers
    const int e = min(r & 0xffff, E - 1);
    const int c = (r >> 16) & cmask;
    return (uint32_t)(e + c * (Ep + second_slot<W>(e) - e)) * W * 4;
  };
  uint32_t offp[HE][2];
#pragma unroll
  for (int h = 0; h < HE; ++h)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t o0 = owner ? slot_bytes(ridx[h * G32 + j + 2 * q]) : 0u;
      const uint32_t o1 = owner ? slot_bytes(ridx[h * G32 + j + 2 * q + 1]) : 0u;
      offp[h][q] = o0 | o1 << 16;
    }
  // cost table of step t into buffer t & 1 (copies Ep W floats each): row w of entry e at [(t & 1) B + e W + w],
  // and with two copies also at [(t & 1) B + (Ep + second_slot(e)) W + w]
  // (with one copy the second store repeats the first: a branch there costs the loop 20 registers)
  const int B = copies * Ep * W;
  const int second = copies == 2 ? (Ep + second_slot<W>(tid)) * W : tid * W;
  // x_t from the workgroup's LDS copy of the sequence (a global load here would put its latency on every
  // step's critical path, between the evaluations and the barrier)
  auto fill = [&](int t) {
    if (tid < E) {
      const int tt = t + roll < g.steps ? t + roll : t + roll - g.steps;  // roll < steps
      const float x0 = ((lds_cf)xs)[tt * V];
      const float x1 = V == 2 ? ((lds_cf)xs)[tt * V + 1] : 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float d0 = urow[w][0] - x0;
        float c = d0 * d0;
        if constexpr (V == 2) {
          const float d1 = urow[w][V - 1] - x1;
          c = c + d1 * d1;
        }
        ((lds_f)ctab)[(t & 1) * B + tid * W + w] = c;
        ((lds_f)ctab)[(t & 1) * B + second + w] = c;
      }
    }
  };
  // one step; the first (no predecessor minima, the overlap mask) written apart from the loop of the others, so
  // that the loop holds one version of the evaluations whatever the compiler makes of the rest
  auto step = [&](int t, auto first_c) __attribute__((always_inline)) {
    constexpr bool first = decltype(first_c)::value;
    // 32-bit LDS indices: 64-bit ones take scalar register pairs, and at more than 80 scalar registers (with
    // the trap handler's) two 1024-thread workgroups no longer fit a CU
    lds_cf prev = (lds_cf)(first ? prev_lds : prev_lds + ((t - 1) & 1) * G32);
    lds_f cur = (lds_f)(prev_lds + (t & 1) * G32);
    // the cost tables sit at the start of the workgroup's LDS: byte address = buffer base + offset
    const uint32_t cbase = (uint32_t)((t & 1) * B * 4);
    auto groups = [&]() {
      // the step's history row, addressed before the loop (the store after it is the only branch)
      float4* hrow = reinterpret_cast<float4*>(hist + (int64_t)t * g.G + j);
      float best[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) best[e] = inf;
      // the predecessor group of state h G + j is h (G >> kv) + (j >> kv) (G is a multiple of 2^kv).  With
      // G >> kv known at compile time (PS) the reads take immediate offsets; otherwise they go through a
      // pointer per w advanced by G >> kv at every h (opaque, so that the compiler does not turn the advances
      // into one scalar register per (h, w): 15 of them would put the kernel past 80)
      const int pstride = PS ? PS : G32 >> kv, pj = j >> kv;
      lds_cf pp[W];
#pragma unroll
      for (int w = 0; w < W; ++w) pp[w] = prev + w * HE * pstride + pj;
      // costs of entry h's four groups, read one h ahead: the reads of h + 1 are in flight while h is evaluated
      auto read_costs = [&](int h, float (&c)[4][W]) __attribute__((always_inline)) {
        // opaque here, so that the halves are extracted at their use instead of unpacked into 4 HE registers
        // ahead of the loop
        asm volatile("" : "+v"(offp[h][0]), "+v"(offp[h][1]));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t ob = cbase + ((e & 1) ? offp[h][e >> 1] >> 16 : offp[h][e >> 1] & 0xffffu);
          if constexpr (W == 2) {
            const f2v c2 = *(lds_cf2)((lds_cb)ctab + ob);
            c[e][0] = c2.x;
            c[e][1] = c2.y;
          } else {
            c[e][0] = *(lds_cf)((lds_cb)ctab + ob);
          }
        }
      };
      // entries read ahead (2, 3 or 7 ahead, or no schedule barrier below: the same time within 3%)
      constexpr int PD = 1;
      float cc[PD + 1][4][W];
#pragma unroll
      for (int h = 0; h < PD && h < HE; ++h) read_costs(h, cc[h]);
#pragma unroll
      for (int h = 0; h < HE; ++h) {
        if (h + PD < HE) read_costs(h + PD, cc[(h + PD) % (PD + 1)]);
#pragma unroll
        for (int w = 0; w < W; ++w) {
          const int ps = (h + w * HE) * pstride + pj;  // state (h + w HE) G + j
          float pv = 0.f;
          if constexpr (!first) {
            if constexpr (PS != 0) {
              pv = pp[0][(h + w * HE) * PS];
            } else {
              pv = *pp[w];
              pp[w] += pstride;
              asm volatile("" : "+v"(pp[w]));
            }
          }
          const bool masked_out = first && masked && ps != overlap;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = cc[h % (PD + 1)][e][w];
            if constexpr (first)
              v = masked_out ? inf : v;
            else
              v = pv + v;
            best[e] = fmin(v, best[e]);
          }
        }
        // one h at a time: left alone, the scheduler issues the reads of all HE entries at once and runs out
        // of registers (spills)
        __builtin_amdgcn_sched_barrier(0);
      }
      const float4 b4 = make_float4(best[0], best[1], best[2], best[3]);
      *(lds_f4)(cur + j) = f4v{b4.x, b4.y, b4.z, b4.w};
      if (live) *hrow = b4;
    };
    if (owner) groups();
    // the next step's cost table (the last step's costs come from the table itself, in final_argmin)
    if (t + 2 < g.steps) fill(t + 1);
    __syncthreads();
  };
  fill(0);
  __syncthreads();
  if (g.steps > 1) step(0, std::true_type{});
  for (int t = 1; t + 1 < g.steps; ++t) step(t, std::false_type{});
  const Sequence<float, V> seqs[1] = {sq};
  float* const hists[1] = {hist};
  const int64_t ovs[1] = {overlap};
  final_argmin<float, V, 1>(seqs, table, hists, prev_lds, g, roll, masked, ovs, best_state, red_v, red_i);
}

// Walk back from the last state to step `stop` with wave 0: returns the state at `stop`, and writes
// the values (times scale) and states of steps [stop, steps) if out / states_out are given.
template <typename T, int V>
__device__ int64_t backtrack(const Sequence<T, V>& seq, const T* __restrict__ table, const T* __restrict__ hist,
                             const SearchGeom& g, int roll, bool masked, int64_t overlap, int64_t state, int stop,
                             T scale, T* __restrict__ out, int64_t* __restrict__ states_out) {
  const int lane = threadIdx.x & 63;
  const int64_t G = g.G, H = (int64_t)1 << g.KV;
  const T inf = inf_value<T>();
  for (int t = g.steps - 1; t > stop; --t) {
    if (lane == 0) {
      if (out)
        for (int v = 0; v < V; ++v) out[(int64_t)t * V + v] = table[state * V + v] * scale;
      if (states_out) states_out[t] = state;
    }
    const int64_t low = state >> g.KV;
    T x0, x1;
    seq.at(t - 1, roll, x0, x1);
    T bv = inf;
    int64_t bi = INT64_MAX;
    for (int64_t h = lane; h < H; h += 64) {
      const int64_t s = h * G + low;
      T c = local_cost<T, V>(table, s, x0, x1);
      if (t - 1 >= 1) {
        c = hist[(int64_t)(t - 2) * G + (s >> g.KV)] + c;
      } else if (masked && (s >> g.KV) != overlap) {
        c = inf;
      }
      if (c < bv || bi == INT64_MAX) {
        bv = c;
        bi = h;
      }
    }
    wave_argmin(bv, bi);
    state = (bi * G + low) & ((G << g.KV) - 1);
  }
  if (lane == 0) {
    if (out)
      for (int v = 0; v < V; ++v) out[(int64_t)stop * V + v] = table[state * V + v] * scale;
    if (states_out) states_out[stop] = state;
  }
  return state;
}

// NS sequences per workgroup: rows NS blockIdx.x + k; wave k walks sequence k back.
template <typename T, int V, int NS>
__global__ __launch_bounds__(VT_THREADS) void viterbi_kernel(const T* __restrict__ x, const T* __restrict__ table,
                                                             T* __restrict__ hist_all, const T* __restrict__ scale,
                                                             T* __restrict__ out, int64_t* __restrict__ states,
                                                             int64_t rows, int L, int KV, int steps, int tail_biting,
                                                             int prev_in_lds, int vec4) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ T red_v[NS * (VT_THREADS / 64)];
  __shared__ int64_t red_i[NS * (VT_THREADS / 64)];
  __shared__ int64_t sh_state[NS], sh_overlap[NS];
  SearchGeom g{L, KV, steps, (int64_t)1 << (L - KV), vec4 != 0};
  Sequence<T, V> seq[NS];
  bool live[NS];
  T* hist[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const int64_t row = (int64_t)blockIdx.x * NS + k;
    live[k] = row < rows;
    const int64_t r = live[k] ? row : rows - 1;  // a valid stand-in for the reads
    seq[k] = Sequence<T, V>{x + r * (int64_t)steps * V, steps};
    hist[k] = hist_all + r * (int64_t)(steps > 1 ? steps - 1 : 1) * g.G;
  }
  T* prev_lds = prev_in_lds ? reinterpret_cast<T*>(smem) : nullptr;
  const int wave = threadIdx.x >> 6;
  int64_t overlap[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) overlap[k] = 0;
  if (tail_biting) {
    const int half = steps / 2;
    forward_pass<T, V, NS>(seq, live, table, hist, prev_lds, g, steps - half, false, overlap, sh_state, red_v, red_i);
#pragma unroll
    for (int k = 0; k < NS; ++k)
      if (wave == k && live[k]) {
        const int64_t st = backtrack<T, V>(seq[k], table, hist[k], g, steps - half, false, 0, sh_state[k], half, T(1),
                                           nullptr, nullptr);
        if ((threadIdx.x & 63) == 0) sh_overlap[k] = st >> KV;
      }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NS; ++k) overlap[k] = live[k] ? sh_overlap[k] : 0;
  }
  forward_pass<T, V, NS>(seq, live, table, hist, prev_lds, g, 0, tail_biting != 0, overlap, sh_state, red_v, red_i);
#pragma unroll
  for (int k = 0; k < NS; ++k)
    if (wave == k && live[k]) {
      const int64_t row = (int64_t)blockIdx.x * NS + k;
      const T sc = scale ? scale[row] : T(1);
      T* orow = out ? out + row * (int64_t)steps * V : nullptr;
      int64_t* srow = states ? states + row * (int64_t)steps : nullptr;
      backtrack<T, V>(seq[k], table, hist[k], g, 0, tail_biting != 0, overlap[k], sh_state[k], 0, sc, orow, srow);
    }
}

// viterbi_kernel with the forward passes of forward_rows (fp32, one sequence per workgroup; G <= 4 VT_THREADS,
// G % 4 == 0, 2^KV == H, E <= ROWS_MAX; the previous minima always in LDS).  Dynamic LDS: the cost tables
// (2 x copies x Ep x W floats, Ep = E for one copy, E rounded up to a row of 64 / W entries for two; at LDS
// address 0 so that a 16-bit byte offset addresses them), the minima (2 G floats), then the sequence (steps V
// floats).
template <int V, int H, int W, int PS>
__global__ __launch_bounds__(VT_THREADS) void viterbi_rows_kernel(const float* __restrict__ x,
                                                                  const float* __restrict__ table,
                                                                  const float* __restrict__ urows,
                                                                  const int* __restrict__ ridx, int E, int Ep,
                                                                  int copies, float* __restrict__ hist_all,
                                                                  const float* __restrict__ scale,
                                                                  float* __restrict__ out,
                                                                  int64_t* __restrict__ states, int64_t rows, int L,
                                                                  int KV, int steps, int tail_biting) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ float red_v[VT_THREADS / 64];
  __shared__ int64_t red_i[VT_THREADS / 64];
  __shared__ int64_t sh_state[1], sh_overlap;
  SearchGeom g{L, KV, steps, (int64_t)1 << (L - KV), true};
  const int64_t row = blockIdx.x;
  const Sequence<float, V> sq{x + row * (int64_t)steps * V, steps};
  float* hist = hist_all + row * (int64_t)(steps > 1 ? steps - 1 : 1) * g.G;
  float* ctab = reinterpret_cast<float*>(smem);
  float* prev_lds = ctab + ((2 * copies * Ep * W + 3) & ~3);
  float* xs = prev_lds + 2 * g.G;  // the sequence, steps V floats
  for (int i = threadIdx.x; i < steps * V; i += VT_THREADS) xs[i] = sq.x[i];
  __syncthreads();  // the copy before any thread's first cost-table fill
  // this thread's entry (the cost table entry it evaluates each step)
  float urow[W][V];
#pragma unroll
  for (int w = 0; w < W; ++w)
#pragma unroll
    for (int v = 0; v < V; ++v) urow[w][v] = (int)threadIdx.x < E ? urows[(threadIdx.x * W + w) * V + v] : 0.f;
  const bool wave0 = threadIdx.x < 64;
  int64_t overlap = 0;
  if (tail_biting) {
    const int half = steps / 2;
    forward_rows<V, H, W, PS>(sq, xs, true, table, urow, E, Ep, copies, ridx, ctab, hist, prev_lds, g, steps - half,
                          false, 0, sh_state, red_v, red_i);
    if (wave0) {
      const int64_t st = backtrack<float, V>(sq, table, hist, g, steps - half, false, 0, sh_state[0], half, 1.f,
                                             nullptr, nullptr);
      if (threadIdx.x == 0) sh_overlap = st >> KV;
    }
    __syncthreads();
    overlap = sh_overlap;
  }
  forward_rows<V, H, W, PS>(sq, xs, true, table, urow, E, Ep, copies, ridx, ctab, hist, prev_lds, g, 0, tail_biting != 0,
                        overlap, sh_state, red_v, red_i);
  if (wave0) {
    const float sc = scale ? scale[row] : 1.f;
    float* orow = out ? out + row * (int64_t)steps * V : nullptr;
    int64_t* srow = states ? states + row * (int64_t)steps : nullptr;
    backtrack<float, V>(sq, table, hist, g, 0, tail_biting != 0, overlap, sh_state[0], 0, sc, orow, srow);
  }
}

template <int V, int H, int W, int PS>
void launch_viterbi_rows(size_t lds, hipStream_t stream, const float* x, const float* table, const float* urows,
                         const int* ridx, int E, int Ep, int copies, float* hist, const float* scale, float* out,
                         int64_t* states, int64_t rows, int L, int KV, int steps, int tail_biting) {
  hipLaunchKernelGGL((viterbi_rows_kernel<V, H, W, PS>), dim3((unsigned)rows), dim3(VT_THREADS), lds, stream, x, table,
                     urows, ridx, E, Ep, copies, hist, scale, out, states, rows, L, KV, steps, tail_biting);
}

template <int V, int W>
void launch_viterbi_rows_h(int H, size_t lds, hipStream_t stream, const float* x, const float* table,
                           const float* urows, const int* ridx, int E, int Ep, int copies, float* hist,
                           const float* scale, float* out, int64_t* states, int64_t rows, int L, int KV, int steps,
                           int tail_biting) {
  auto go = [&](auto kernel_h, auto kernel_ps) {
    constexpr int HH = decltype(kernel_h)::value, PS = decltype(kernel_ps)::value;
    launch_viterbi_rows<V, HH, W, PS>(lds, stream, x, table, urows, ridx, E, Ep, copies, hist, scale, out, states,
                                      rows, L, KV, steps, tail_biting);
  };
  using rt = std::integral_constant<int, 0>;
  if (H == 4)
    go(std::integral_constant<int, 4>{}, rt{});
  else if (H == 8)
    go(std::integral_constant<int, 8>{}, rt{});
  else if (L == 16)  // HYB and 1MAD at L = 16, K V = 4: the predecessor stride 2^(L - 2 K V) = 256 at compile time
    go(std::integral_constant<int, 16>{}, std::integral_constant<int, 256>{});
  else
    go(std::integral_constant<int, 16>{}, rt{});
}

template <typename T, int V, int NS>
void launch_viterbi(size_t lds, bool in_lds, hipStream_t stream, const T* x, const T* table, T* hist, const T* scale,
                    T* out, int64_t* states, int64_t rows, int L, int KV, int steps, int tail_biting) {
  const dim3 grid((unsigned)((rows + NS - 1) / NS));
  const bool vec4 = sizeof(T) == 4 && L - KV >= 2 && KV >= 2 && ((uintptr_t)table & 15) == 0 &&
                    ((uintptr_t)hist & 15) == 0;
  hipLaunchKernelGGL((viterbi_kernel<T, V, NS>), grid, dim3(VT_THREADS), in_lds ? lds : 0, stream, x, table, hist,
                     scale, out, states, rows, L, KV, steps, tail_biting, in_lds ? 1 : 0, vec4 ? 1 : 0);
}

template <typename T>
int viterbi(const T* x, const T* table, T* hist, const T* scale, T* out, int64_t* states, int64_t rows, int64_t steps,
            int L, int K, int V, int tail_biting, hipStream_t stream) {
  const int KV = K * V;
  if (rows < 0 || steps < 1 || L < 1 || L > 24 || K < 1 || (V != 1 && V != 2) || KV > L || KV > 8) return GPTQ2D_EINVAL;
  if (rows == 0) return 0;
  if (rows > 0x7fffffff || steps > 0x7fffffff) return GPTQ2D_EUNSUPPORTED;
  const int64_t G = (int64_t)1 << (L - KV);
  // two sequences per workgroup (each table load serves both) when their minima fit in LDS and one per
  // workgroup would put more workgroups than compute units on the chip: a CU then runs two of them at half
  // speed each (C4's calls of 257 to 511 sequences: 2.8-2.9 ms with one sequence per workgroup, 1.8-1.9 ms
  // with two), else one
  const size_t lds1 = 2 * G * sizeof(T), lds2 = 2 * lds1;
  const bool two = lds2 <= 96 * 1024 && rows > device_cus();
  const size_t lds = two ? lds2 : lds1;
  const bool in_lds = lds <= 96 * 1024;
  if (two) {
    if (V == 1)
      launch_viterbi<T, 1, 2>(lds, in_lds, stream, x, table, hist, scale, out, states, rows, L, KV, (int)steps,
                              tail_biting);
    else
      launch_viterbi<T, 2, 2>(lds, in_lds, stream, x, table, hist, scale, out, states, rows, L, KV, (int)steps,
                              tail_biting);
  } else {
    if (V == 1)
      launch_viterbi<T, 1, 1>(lds, in_lds, stream, x, table, hist, scale, out, states, rows, L, KV, (int)steps,
                              tail_biting);
    else
      launch_viterbi<T, 2, 1>(lds, in_lds, stream, x, table, hist, scale, out, states, rows, L, KV, (int)steps,
                              tail_biting);
  }
  return (int)hipGetLastError();
}

// The search with the cost tables of the distinct rows (W = 1) or row pairs (W = 2) where it applies (fp32,
// 2 <= KV <= 4, G % 4 == 0 and G % 2^KV == 0, G <= 4 VT_THREADS, 1 <= E <= ROWS_MAX, 16-byte aligned table and
// history, LDS for the minima and the cost tables), else the plain search.  Same results either way.
int viterbi_rows(const float* x, const float* table, const float* urows, const int* ridx, int64_t E, int W,
                 float* hist, const float* scale, float* out, int64_t* states, int64_t rows, int64_t steps, int L,
                 int K, int V, int tail_biting, hipStream_t stream) {
  const int KV = K * V;
  if (rows < 0 || steps < 1 || L < 1 || L > 24 || K < 1 || (V != 1 && V != 2) || KV > L || KV > 8) return GPTQ2D_EINVAL;
  if (rows == 0) return 0;
  if (rows > 0x7fffffff || steps > 0x7fffffff) return GPTQ2D_EUNSUPPORTED;
  const int64_t G = (int64_t)1 << (L - KV);
  const bool shape_ok = urows && ridx && (W == 1 || W == 2) && E >= 1 && E <= ROWS_MAX && KV >= 2 && KV <= 4 &&
                        G % 4 == 0 && G % (1 << KV) == 0 && G <= 4 * VT_THREADS && ((uintptr_t)table & 15) == 0 &&
                        ((uintptr_t)hist & 15) == 0;
  // one sequence per workgroup: with two, the compiler spills the evaluation loop (two sequences' costs and
  // minima beside the offsets exceed the 128 registers of a 1024-thread workgroup); more rows than compute
  // units queue as further rounds.  Two copies of the cost table where they fit beside a second workgroup on
  // the CU (160 KB of LDS), or where one copy does not leave room for it either.
  const int NB = 64 / W;
  const int64_t Ep2 = (E + NB - 1) / NB * NB;
  auto lds_of = [&](int64_t copies, int64_t ep) {
    return (size_t)2 * G * 4 + (size_t)((2 * copies * ep * W + 3) & ~3) * 4 + (size_t)steps * V * 4;
  };
  constexpr size_t two_per_cu = 78 * 1024, most = 96 * 1024;
  const bool two = lds_of(2, Ep2) <= most && (lds_of(2, Ep2) <= two_per_cu || lds_of(1, E) > two_per_cu);
  const int copies = two ? 2 : 1;
  const int Ep = (int)(two ? Ep2 : E);
  const size_t lds = lds_of(copies, Ep);
  if (!shape_ok || lds > most)
    return viterbi<float>(x, table, hist, scale, out, states, rows, steps, L, K, V, tail_biting, stream);
  const int H = 1 << KV;
  const int Ei = (int)E;
  if (W == 2) {
    if (V == 1)
      launch_viterbi_rows_h<1, 2>(H, lds, stream, x, table, urows, ridx, Ei, Ep, copies, hist, scale, out, states,
                                  rows, L, KV, (int)steps, tail_biting);
    else
      launch_viterbi_rows_h<2, 2>(H, lds, stream, x, table, urows, ridx, Ei, Ep, copies, hist, scale, out, states,
                                  rows, L, KV, (int)steps, tail_biting);
  } else {
    if (V == 1)
      launch_viterbi_rows_h<1, 1>(H, lds, stream, x, table, urows, ridx, Ei, Ep, copies, hist, scale, out, states,
                                  rows, L, KV, (int)steps, tail_biting);
    else
      launch_viterbi_rows_h<2, 1>(H, lds, stream, x, table, urows, ridx, Ei, Ep, copies, hist, scale, out, states,
                                  rows, L, KV, (int)steps, tail_biting);
  }
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

// Size in elements of the history workspace for `rows` sequences of `steps` steps.
int64_t gptq2d_viterbi_workspace(int64_t rows, int64_t steps, int32_t L, int32_t K, int32_t V) {
  if (rows < 0 || steps < 1 || K * V > L) return -1;
  return rows * (steps > 1 ? steps - 1 : 1) * ((int64_t)1 << (L - K * V));
}

#define GPTQ2D_VITERBI_ABI(SUF, T)                                                                                  \
  int gptq2d_viterbi_##SUF(const T* x, const T* table, T* hist, const T* scale, T* out, int64_t* states,           \
                           int64_t rows, int64_t steps, int32_t L, int32_t K, int32_t V, int32_t tail_biting,      \
                           hipStream_t stream) {                                                                   \
    return viterbi<T>(x, table, hist, scale, out, states, rows, steps, L, K, V, tail_biting, stream);                \
  }

GPTQ2D_VITERBI_ABI(f32, float)
GPTQ2D_VITERBI_ABI(f64, double)

// The fp32 search over a table given as entries of its distinct rows or row pairs (see viterbi_rows).
int gptq2d_viterbi_rows_f32(const float* x, const float* table, const float* urows, const int32_t* ridx, int64_t E,
                            int32_t W, float* hist, const float* scale, float* out, int64_t* states, int64_t rows,
                            int64_t steps, int32_t L, int32_t K, int32_t V, int32_t tail_biting, hipStream_t stream) {
  return viterbi_rows(x, table, urows, ridx, E, W, hist, scale, out, states, rows, steps, L, K, V, tail_biting,
                      stream);
}

}  // extern "C"
