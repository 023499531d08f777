// Packed output formats of a quantized layer (no counterpart kernels in the reference, which returns only
// dequantized values; quantizer_trellis.py:11-16 states that the T*K-bit code is recoverable).
//
// INT codes.  Under the affine quantizer (quantizer_int.py:63-83) an entry's value is z = (q - zp) * s with an
// integer code q in [qmin, qmax].  Its packed code is u = q - qmin in `bits` = ceil(log2(qmax - qmin + 1))
// bits; the codes of a row of the [B, m, n] layer form one little-endian bit field: code j occupies bits
// [j*bits, (j+1)*bits) of the row, bit k of the row is bit (k % 32) of word k / 32 (for 4 bits: code j is
// nibble j % 8 of word j / 8, low nibble first).  Rows start on a word boundary (row_words words each, the
// unused tail zero).  The packer recovers q = rint(z / s + zp) and counts, per row, the entries whose
// value is not reproduced by (q - zp) * s with q in range (those are packed as code 0); the
// unpacker evaluates (q - zp) * s, the quantizer's own expression, so a counted-clean row round-trips
// exactly (as numbers; the sign of a zero is not kept).  Scale and zero point are read through element
// strides (0 broadcasts).
//
// Trellis streams.  A bitshift-trellis path (quantizer_trellis.py:82-143) of S = T / V states of L bits
// shifts K*V new bits into the low end of the state each step: s_{t+1} >> KV == s_t mod 2^(L - KV).  Its
// stream holds the top KV bits of every state in order, MSB first (stream bit k is bit 31 - k % 32 of word
// k / 32), so state t is the L-bit window starting at stream bit t*KV.  A tail-biting path is circular
// (s_0 >> KV == s_{S-1} mod 2^(L-KV)): exactly T*K bits, windows read modulo that length.  Without tail-biting
// the stream adds the low L - KV bits of the last state (T*K + L - KV bits).  The packer counts, per
// sequence, states out of range, breaks of the shift rule and copies of a state that disagree; the decoder
// writes the states and/or the values table[s, v] * scale, the quantizer's expression.
//
// Sequences are the p x q super-entries of a [B, m, n] layout read row by row (the layout of the trellis
// quantizer's super-entries); step t of sequence (b, I, J) holds entries e = t*V .. t*V + V - 1 of the block,
// entry e at (I*p + e / q, J*q + e % q).  A plain [R, T] array of sequences is the case B = 1, m = R,
// n = T, p = 1, q = T.  In the packer the per-entry state map may repeat each state over its V entries
// (copies = V) or list the states once per step (copies = 1, entry e = t).
#include "common.h"

namespace {

constexpr int PACK_WAVES = 4;

// Packed code of value zv under (s, zp); ok = the quantizer's output for that code equals zv (as numbers: the
// quantizer gives -0 for a code of -0, which rint returns for small negative inputs; a zero's sign is not kept).
template <typename T>
__device__ __forceinline__ uint32_t int_code(T zv, T s, T zp, T qmin, T qmax, bool& ok) {
  const T q = round_even(zv / s + zp);
  ok = q >= qmin && q <= qmax && (q - zp) * s == zv;
  return ok ? (uint32_t)(int64_t)(q - qmin) : 0u;
}

template <typename T>
struct IntLayout {
  const T* s;
  int64_t sb, sm, sn;
  const T* zp;
  int64_t zb, zm, zn;
};

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int k = 32; k >= 1; k >>= 1) v += __shfl_xor(v, k, 64);
  return v;
}

// One wave per row.  POW2 (bits divides 32): lane = code, the 32 / bits codes of a word OR-reduced across
// lanes; otherwise lane = word, gathering the codes that overlap it.
template <typename T, bool POW2>
__global__ __launch_bounds__(64 * PACK_WAVES) void int_pack_kernel(const T* __restrict__ z, int64_t rows, int64_t m,
                                                                    int64_t n, IntLayout<T> lay, T qmin, T qmax,
                                                                    int bits, uint32_t* __restrict__ words,
                                                                    int64_t row_words, int32_t* __restrict__ bad) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * PACK_WAVES + (threadIdx.x >> 6);
  if (row >= rows) return;  // uniform over the wave
  const int64_t b = row / m, i = row % m;
  const T* zr = z + row * n;
  const T* sr = lay.s + b * lay.sb + i * lay.sm;
  const T* pr = lay.zp ? lay.zp + b * lay.zb + i * lay.zm : nullptr;
  uint32_t* wr = words + row * row_words;
  int nbad = 0;
  if constexpr (POW2) {
    const int per = 32 / bits;  // codes per word, a power of two dividing 64
    const int64_t used = cdiv(n, per);
    for (int64_t j0 = 0; j0 < row_words * per; j0 += 64) {
      const int64_t j = j0 + lane;
      uint32_t v = 0;
      if (j < n) {
        bool ok;
        v = int_code(zr[j], sr[j * lay.sn], pr ? pr[j * lay.zn] : T(0), qmin, qmax, ok) << ((lane % per) * bits);
        nbad += ok ? 0 : 1;
      }
      for (int k = 1; k < per; k <<= 1) v |= __shfl_xor(v, k, 64);
      const int64_t w = j / per;
      if (lane % per == 0 && w < row_words) wr[w] = w < used ? v : 0u;
    }
  } else {
    const int64_t nbits = n * bits;
    for (int64_t w = lane; w < row_words; w += 64) {
      uint64_t acc = 0;
      const int64_t first = w * 32;
      if (first < nbits) {
        const int64_t j0 = first / bits;
        const int64_t j1 = min(n, cdiv(first + 32, bits));
        for (int64_t j = j0; j < j1; ++j) {
          bool ok;
          const uint64_t u = int_code(zr[j], sr[j * lay.sn], pr ? pr[j * lay.zn] : T(0), qmin, qmax, ok);
          const int64_t off = j * bits - first;  // in (-bits, 32)
          if (off >= 0) {
            acc |= u << off;
            nbad += ok ? 0 : 1;  // counted in the word where the code starts
          } else {
            acc |= u >> (-off);
          }
        }
      }
      wr[w] = (uint32_t)acc;
    }
  }
  nbad = wave_sum(nbad);
  if (lane == 0 && bad) bad[row] = nbad;
}

template <typename T>
__global__ __launch_bounds__(256) void int_unpack_kernel(const uint32_t* __restrict__ words, int64_t rows, int64_t m,
                                                         int64_t n, int64_t row_words, IntLayout<T> lay, T qmin,
                                                         int bits, T* __restrict__ z) {
  const int64_t total = rows * n;
  const uint32_t mask = bits == 32 ? 0xffffffffu : ((1u << bits) - 1u);
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int64_t row = idx / n, j = idx % n;
    const int64_t b = row / m, i = row % m;
    const uint32_t* wr = words + row * row_words;
    const int64_t start = j * bits;
    const int64_t w = start >> 5;
    const int off = (int)(start & 31);
    uint64_t v = wr[w] >> off;
    if (off + bits > 32) v |= (uint64_t)wr[w + 1] << (32 - off);
    const T q = T((uint32_t)v & mask) + qmin;
    const T s = lay.s[b * lay.sb + i * lay.sm + j * lay.sn];
    const T zp = lay.zp ? lay.zp[b * lay.zb + i * lay.zm + j * lay.zn] : T(0);
    z[idx] = (q - zp) * s;
  }
}

// ------------------------------------------------------------------------------------------------ trellis

struct SeqLayout {
  int64_t m, n, p, q;  // the [B, m, n] layout of p x q blocks
  int64_t ncol;        // n / q
  int64_t per_b;       // (m / p) * (n / q) sequences per batch matrix

  // Offset of entry e of sequence r.
  __device__ __forceinline__ int64_t at(int64_t r, int64_t e) const {
    const int64_t b = r / per_b, k = r % per_b;
    const int64_t I = k / ncol, J = k % ncol;
    return (b * m + I * p + e / q) * n + J * q + e % q;
  }
};

// MSB-first bit writer into one sequence's words.
struct StreamWriter {
  uint32_t* w;
  int64_t pos = 0;  // words written
  uint64_t acc = 0;
  int nacc = 0;

  __device__ __forceinline__ void put(uint32_t v, int k) {  // the low k <= 32 bits of v
    acc = (acc << k) | (k == 32 ? (uint64_t)v : ((uint64_t)v & ((1ull << k) - 1)));
    nacc += k;
    if (nacc >= 32) {
      w[pos++] = (uint32_t)(acc >> (nacc - 32));
      nacc -= 32;
    }
  }
  __device__ __forceinline__ void flush(int64_t row_words) {
    if (nacc > 0) w[pos++] = (uint32_t)(acc << (32 - nacc));
    nacc = 0;
    while (pos < row_words) w[pos++] = 0u;
  }
};

// One thread per sequence.
__global__ __launch_bounds__(256) void trellis_pack_kernel(const int64_t* __restrict__ st, int64_t seqs, SeqLayout lay,
                                                           int64_t steps, int copies, int L, int KV, int tail,
                                                           uint32_t* __restrict__ words, int64_t row_words,
                                                           int32_t* __restrict__ bad) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= seqs) return;
  const int64_t low_mask = ((int64_t)1 << (L - KV)) - 1;
  const int64_t limit = (int64_t)1 << L;
  StreamWriter out{words + r * row_words};
  int nbad = 0;
  int64_t first = 0, prev = 0;
  for (int64_t t = 0; t < steps; ++t) {
    int64_t s = st[lay.at(r, t * copies)];
    for (int c = 1; c < copies; ++c) nbad += st[lay.at(r, t * copies + c)] != s ? 1 : 0;
    if (s < 0 || s >= limit) {
      ++nbad;
      s = 0;
    }
    if (t == 0)
      first = s;
    else
      nbad += (s >> KV) != (prev & low_mask) ? 1 : 0;
    out.put((uint32_t)(s >> (L - KV)), KV);
    prev = s;
  }
  if (tail) {
    nbad += (first >> KV) != (prev & low_mask) ? 1 : 0;
  } else {
    for (int k = L - KV; k > 0; k -= 32 < k ? 32 : k) {
      const int c = k < 32 ? k : 32;
      out.put((uint32_t)(prev >> (k - c)), c);
    }
  }
  out.flush(row_words);
  if (bad) bad[r] = nbad;
}

__device__ __forceinline__ uint32_t stream_bit(const uint32_t* w, int64_t k) { return (w[k >> 5] >> (31 - (k & 31))) & 1u; }

// One thread per (sequence, step): the state is the L-bit window at bit t*KV (modulo the stream length for
// a tail-biting path); states [seqs, steps] and/or values in the block layout.
template <typename T>
__global__ __launch_bounds__(256) void trellis_unpack_kernel(const uint32_t* __restrict__ words, int64_t seqs,
                                                             SeqLayout lay, int64_t steps, int64_t row_words, int L,
                                                             int KV, int V, int tail, const T* __restrict__ table,
                                                             const T* __restrict__ scale, int64_t scale_stride,
                                                             T* __restrict__ values, int64_t* __restrict__ states) {
  const int64_t total = seqs * steps;
  const int64_t len = tail ? steps * KV : steps * KV + L - KV;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int64_t r = idx / steps, t = idx % steps;
    const uint32_t* w = words + r * row_words;
    const int64_t start = t * KV;
    int64_t s = 0;
    if (start + L <= len) {
      const int64_t wi = start >> 5;
      const int off = (int)(start & 31);
      uint64_t v = (uint64_t)w[wi] << 32;
      if (off + L > 32) v |= w[wi + 1];
      s = (int64_t)((v >> (64 - off - L)) & ((1ull << L) - 1));
    } else {  // a tail-biting window that wraps
      for (int i = 0; i < L; ++i) s = (s << 1) | stream_bit(w, (start + i) % len);
    }
    if (states) states[idx] = s;
    if (values) {
      const T sc = scale ? scale[r * scale_stride] : T(1);
      for (int v = 0; v < V; ++v) values[lay.at(r, t * V + v)] = table[s * V + v] * sc;
    }
  }
}

bool make_layout(SeqLayout& lay, int64_t B, int64_t m, int64_t n, int64_t p, int64_t q, int64_t& seqs) {
  if (B < 0 || m < 0 || n < 0 || p <= 0 || q <= 0 || m % p || n % q) return false;
  lay.m = m;
  lay.n = n;
  lay.p = p;
  lay.q = q;
  lay.ncol = n / q;
  lay.per_b = (m / p) * (n / q);
  seqs = B * lay.per_b;
  return true;
}

bool trellis_shape_ok(int L, int K, int V) { return K >= 1 && V >= 1 && K * V <= L && L <= 30; }

template <typename T>
bool int_layout(IntLayout<T>& lay, const T* s, const int64_t* ss, const T* zp, const int64_t* zs) {
  if (!s || !ss || (zp && !zs)) return false;
  lay.s = s;
  lay.sb = ss[0];
  lay.sm = ss[1];
  lay.sn = ss[2];
  lay.zp = zp;
  lay.zb = zp ? zs[0] : 0;
  lay.zm = zp ? zs[1] : 0;
  lay.zn = zp ? zs[2] : 0;
  return true;
}

unsigned grid_for(int64_t total) {
  const int64_t blocks = cdiv(total, 256);
  return (unsigned)(blocks < 65536 ? (blocks > 0 ? blocks : 1) : 65536);
}

template <typename T>
int pack_int(const T* z, int64_t B, int64_t m, int64_t n, const T* s, const int64_t* ss, const T* zp,
             const int64_t* zs, double qmin, double qmax, int32_t bits, uint32_t* words, int64_t row_words,
             int32_t* bad, hipStream_t stream) {
  IntLayout<T> lay;
  if (B < 0 || m < 0 || n < 0 || bits < 1 || bits > 16 || !(qmin <= qmax) || qmax - qmin >= (double)(1 << bits) ||
      row_words < cdiv(n * bits, 32))
    return GPTQ2D_EINVAL;
  const int64_t rows = B * m;
  if (rows == 0) return 0;
  if (!int_layout(lay, s, ss, zp, zs)) return GPTQ2D_EINVAL;
  const unsigned grid = (unsigned)cdiv(rows, PACK_WAVES);
  if (32 % bits == 0)
    hipLaunchKernelGGL((int_pack_kernel<T, true>), dim3(grid), dim3(64 * PACK_WAVES), 0, stream, z, rows, m, n, lay,
                       (T)qmin, (T)qmax, bits, words, row_words, bad);
  else
    hipLaunchKernelGGL((int_pack_kernel<T, false>), dim3(grid), dim3(64 * PACK_WAVES), 0, stream, z, rows, m, n, lay,
                       (T)qmin, (T)qmax, bits, words, row_words, bad);
  return (int)hipGetLastError();
}

template <typename T>
int unpack_int(const uint32_t* words, int64_t B, int64_t m, int64_t n, int64_t row_words, const T* s,
               const int64_t* ss, const T* zp, const int64_t* zs, double qmin, int32_t bits, T* z,
               hipStream_t stream) {
  IntLayout<T> lay;
  if (B < 0 || m < 0 || n < 0 || bits < 1 || bits > 16 || row_words < cdiv(n * bits, 32)) return GPTQ2D_EINVAL;
  const int64_t total = B * m * n;
  if (total == 0) return 0;
  if (!int_layout(lay, s, ss, zp, zs)) return GPTQ2D_EINVAL;
  hipLaunchKernelGGL(int_unpack_kernel<T>, dim3(grid_for(total)), dim3(256), 0, stream, words, B * m, m, n, row_words,
                     lay, (T)qmin, bits, z);
  return (int)hipGetLastError();
}

template <typename T>
int trellis_unpack(const uint32_t* words, int64_t B, int64_t m, int64_t n, int64_t p, int64_t q, int64_t row_words,
                   int32_t L, int32_t K, int32_t V, int32_t tail, const T* table, const T* scale, int64_t scale_stride,
                   T* values, int64_t* states, hipStream_t stream) {
  SeqLayout lay;
  int64_t seqs;
  if (!make_layout(lay, B, m, n, p, q, seqs) || !trellis_shape_ok(L, K, V) || (p * q) % V || (values && !table))
    return GPTQ2D_EINVAL;
  const int64_t steps = p * q / V, KV = K * V;
  const int64_t len = tail ? steps * KV : steps * KV + L - KV;
  if (row_words < cdiv(len, 32)) return GPTQ2D_EINVAL;
  const int64_t total = seqs * steps;
  if (total == 0) return 0;
  hipLaunchKernelGGL(trellis_unpack_kernel<T>, dim3(grid_for(total)), dim3(256), 0, stream, words, seqs, lay, steps,
                     row_words, L, K * V, V, tail ? 1 : 0, table, scale, scale_stride, values, states);
  return (int)hipGetLastError();
}

}  // namespace

extern "C" {

int32_t gptq2d_int_code_bits(double qmin, double qmax) {
  if (!(qmin <= qmax) || qmin != (double)(int64_t)qmin || qmax != (double)(int64_t)qmax) return -1;
  const double range = qmax - qmin + 1;
  int bits = 1;
  while ((double)((int64_t)1 << bits) < range) ++bits;
  return bits <= 16 ? bits : -1;
}

int64_t gptq2d_trellis_stream_words(int64_t steps, int32_t L, int32_t K, int32_t V, int32_t tail_biting) {
  if (steps < 1 || !trellis_shape_ok(L, K, V)) return -1;
  const int64_t len = tail_biting ? steps * K * V : steps * K * V + L - K * V;
  return cdiv(len, 32);
}

int gptq2d_trellis_pack(const int64_t* states, int64_t B, int64_t m, int64_t n, int64_t p, int64_t q, int32_t copies,
                        int32_t L, int32_t K, int32_t V, int32_t tail_biting, uint32_t* words, int64_t row_words,
                        int32_t* bad, hipStream_t stream) {
  SeqLayout lay;
  int64_t seqs;
  if (!make_layout(lay, B, m, n, p, q, seqs) || !trellis_shape_ok(L, K, V) || copies < 1 || (p * q) % copies)
    return GPTQ2D_EINVAL;
  const int64_t steps = p * q / copies;
  if (row_words < gptq2d_trellis_stream_words(steps, L, K, V, tail_biting)) return GPTQ2D_EINVAL;
  if (seqs == 0) return 0;
  hipLaunchKernelGGL(trellis_pack_kernel, dim3((unsigned)cdiv(seqs, 256)), dim3(256), 0, stream, states, seqs, lay,
                     steps, copies, L, K * V, tail_biting ? 1 : 0, words, row_words, bad);
  return (int)hipGetLastError();
}

#define GPTQ2D_PACK_ABI(SUF, T)                                                                                      \
  int gptq2d_pack_int_##SUF(const T* z, int64_t B, int64_t m, int64_t n, const T* scale, const int64_t* sstride,     \
                            const T* zp, const int64_t* zstride, double qmin, double qmax, int32_t bits,             \
                            uint32_t* words, int64_t row_words, int32_t* bad, hipStream_t stream) {                  \
    return pack_int<T>(z, B, m, n, scale, sstride, zp, zstride, qmin, qmax, bits, words, row_words, bad, stream);   \
  }                                                                                                                   \
  int gptq2d_unpack_int_##SUF(const uint32_t* words, int64_t B, int64_t m, int64_t n, int64_t row_words,             \
                              const T* scale, const int64_t* sstride, const T* zp, const int64_t* zstride,           \
                              double qmin, int32_t bits, T* z, hipStream_t stream) {                                 \
    return unpack_int<T>(words, B, m, n, row_words, scale, sstride, zp, zstride, qmin, bits, z, stream);            \
  }                                                                                                                   \
  int gptq2d_trellis_unpack_##SUF(const uint32_t* words, int64_t B, int64_t m, int64_t n, int64_t p, int64_t q,       \
                                  int64_t row_words, int32_t L, int32_t K, int32_t V, int32_t tail_biting,           \
                                  const T* table, const T* scale, int64_t scale_stride, T* values, int64_t* states,  \
                                  hipStream_t stream) {                                                              \
    return trellis_unpack<T>(words, B, m, n, p, q, row_words, L, K, V, tail_biting, table, scale, scale_stride,      \
                             values, states, stream);                                                                \
  }

GPTQ2D_PACK_ABI(f32, float)
GPTQ2D_PACK_ABI(f64, double)

}  // extern "C"
