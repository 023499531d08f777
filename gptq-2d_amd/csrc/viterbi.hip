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
// One workgroup (1024 threads) per sequence runs every step of both tail-biting passes: the group
// minima of the previous step sit in LDS (double-buffered, or read back from the history when 2 G
// values do not fit), each thread evaluates the 2^KV predecessors of its groups in order, and every
// step's minima are also stored in an HBM history [steps - 1][G] per sequence.  The final argmin is a
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

// Forward pass: history[t][j] = best_t(j) for t < steps - 1; returns (in *state_out, shared) the
// first argmin of cost_{last} under the masks.  prev_lds: 2 G values of LDS or nullptr.
template <typename T, int V>
__device__ void forward_pass(const Sequence<T, V>& seq, const T* __restrict__ table, T* __restrict__ hist,
                             T* prev_lds, const SearchGeom& g, int roll, bool masked, int64_t overlap,
                             int64_t* best_state, T* red_v, int64_t* red_i) {
  const int tid = threadIdx.x;
  const int64_t G = g.G, H = (int64_t)1 << g.KV;
  const T inf = inf_value<T>();
  for (int t = 0; t + 1 < g.steps; ++t) {
    T x0, x1;
    seq.at(t, roll, x0, x1);
    const T* prev = t == 0 ? nullptr : (prev_lds ? prev_lds + ((t - 1) & 1) * G : hist + (int64_t)(t - 1) * G);
    T* cur_lds = prev_lds ? prev_lds + (t & 1) * G : nullptr;
    T* cur_hist = hist + (int64_t)t * G;
    for (int64_t j = tid; j < G; j += VT_THREADS) {
      T best = inf;
      for (int64_t h = 0; h < H; ++h) {
        const int64_t s = h * G + j;
        T c = local_cost<T, V>(table, s, x0, x1);
        if (t == 0) {
          if (masked && (s >> g.KV) != overlap) c = inf;
        } else {
          c = prev[s >> g.KV] + c;
        }
        best = c < best ? c : best;
      }
      cur_hist[j] = best;
      if (cur_lds) cur_lds[j] = best;
    }
    __syncthreads();
  }
  // final step: first argmin over all states
  T x0, x1;
  seq.at(g.steps - 1, roll, x0, x1);
  const int last = g.steps - 1;
  const T* prev = last == 0 ? nullptr : (prev_lds ? prev_lds + ((last - 1) & 1) * G : hist + (int64_t)(last - 1) * G);
  T bv = inf;
  int64_t bi = INT64_MAX;
  const int64_t S = G << g.KV;
  for (int64_t s = tid; s < S; s += VT_THREADS) {
    T c = local_cost<T, V>(table, s, x0, x1);
    if (last == 0) {
      if (masked && (s >> g.KV) != overlap) c = inf;
    } else {
      c = prev[s >> g.KV] + c;
    }
    if (masked && (s & (G - 1)) != overlap) c = inf;
    if (c < bv || bi == INT64_MAX) {  // increasing s per thread: the first, then strictly smaller ones
      bv = c;
      bi = s;
    }
  }
  wave_argmin(bv, bi);
  const int wave = tid >> 6, lane = tid & 63;
  if (lane == 0) {
    red_v[wave] = bv;
    red_i[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    T v = red_v[0];
    int64_t i = red_i[0];
    for (int w = 1; w < VT_THREADS / 64; ++w) arg_better(v, i, red_v[w], red_i[w]);
    *best_state = i & (S - 1);  // every state is a candidate, so i < S; the mask only keeps reads in bounds
  }
  __syncthreads();
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

template <typename T, int V>
__global__ __launch_bounds__(VT_THREADS) void viterbi_kernel(const T* __restrict__ x, const T* __restrict__ table,
                                                             T* __restrict__ hist_all, const T* __restrict__ scale,
                                                             T* __restrict__ out, int64_t* __restrict__ states,
                                                             int L, int KV, int steps, int tail_biting,
                                                             int prev_in_lds) {
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ T red_v[VT_THREADS / 64];
  __shared__ int64_t red_i[VT_THREADS / 64];
  __shared__ int64_t sh_state, sh_overlap;
  const int64_t row = blockIdx.x;
  SearchGeom g{L, KV, steps, (int64_t)1 << (L - KV)};
  Sequence<T, V> seq{x + row * (int64_t)steps * V, steps};
  T* hist = hist_all + row * (int64_t)(steps > 1 ? steps - 1 : 1) * g.G;
  T* prev_lds = prev_in_lds ? reinterpret_cast<T*>(smem) : nullptr;
  const T sc = scale ? scale[row] : T(1);
  T* orow = out ? out + row * (int64_t)steps * V : nullptr;
  int64_t* srow = states ? states + row * (int64_t)steps : nullptr;
  int64_t overlap = 0;
  if (tail_biting) {
    const int half = steps / 2;
    forward_pass<T, V>(seq, table, hist, prev_lds, g, steps - half, false, 0, &sh_state, red_v, red_i);
    if (threadIdx.x < 64) {
      const int64_t st = backtrack<T, V>(seq, table, hist, g, steps - half, false, 0, sh_state, half, T(1), nullptr,
                                         nullptr);
      if (threadIdx.x == 0) sh_overlap = st >> KV;
    }
    __syncthreads();
    overlap = sh_overlap;
  }
  forward_pass<T, V>(seq, table, hist, prev_lds, g, 0, tail_biting != 0, overlap, &sh_state, red_v, red_i);
  if (threadIdx.x < 64)
    backtrack<T, V>(seq, table, hist, g, 0, tail_biting != 0, overlap, sh_state, 0, sc, orow, srow);
}

template <typename T>
int viterbi(const T* x, const T* table, T* hist, const T* scale, T* out, int64_t* states, int64_t rows, int64_t steps,
            int L, int K, int V, int tail_biting, hipStream_t stream) {
  const int KV = K * V;
  if (rows < 0 || steps < 1 || L < 1 || L > 24 || K < 1 || (V != 1 && V != 2) || KV > L || KV > 8) return GPTQ2D_EINVAL;
  if (rows == 0) return 0;
  if (rows > 0x7fffffff || steps > 0x7fffffff) return GPTQ2D_EUNSUPPORTED;
  const int64_t G = (int64_t)1 << (L - KV);
  const size_t lds = 2 * G * sizeof(T);
  const int in_lds = lds <= 96 * 1024;
  const size_t dyn = in_lds ? lds : 0;
  const dim3 grid((unsigned)rows);
  if (V == 1)
    hipLaunchKernelGGL((viterbi_kernel<T, 1>), grid, dim3(VT_THREADS), dyn, stream, x, table, hist, scale, out, states,
                       L, KV, (int)steps, tail_biting, in_lds);
  else
    hipLaunchKernelGGL((viterbi_kernel<T, 2>), grid, dim3(VT_THREADS), dyn, stream, x, table, hist, scale, out, states,
                       L, KV, (int)steps, tail_biting, in_lds);
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

}  // extern "C"
