/* C ABI of libgptq2d.so: the MI355X (gfx950) GPTQ-2D engine.
 *
 * Every entry point takes raw device pointers and int64 sizes, launches HIP kernels on the given
 * stream (a hipStream_t, passed as void*), never allocates device memory, never synchronises
 * with the host, uses no atomics (results are deterministic) and returns 0 on success, a
 * positive hipError_t, or GPTQ2D_EINVAL / GPTQ2D_EUNSUPPORTED / GPTQ2D_ESCRATCH.  The caller owns all
 * memory (the *_noalloc entry point aside, whose scratch is the library's own).
 * Everything except the profiler may be captured in a hipGraph.
 *
 * Layout conventions.  Y, C and E are contiguous row-major [B, m, n] with B the product of the
 * broadcast batch shape.  L [*, m, m], U [*, n, n] and full-matrix quantizer inputs [*, m, n] may
 * broadcast over the batch: `bnd` is the number of batch dimensions, `bshape[bnd]` the broadcast
 * batch shape and `<x>_stride[bnd]` the operand's batch strides in elements (0 where it broadcasts).
 * L is read only strictly below its (p x p block) diagonal and U only strictly above its (q x q
 * block) diagonal; the other entries may hold anything, NaN included.
 *
 * Every compute entry point exists for float (suffix _f32) and double (suffix _f64); T below is
 * that element type.  The reference (IST-DASLab/GPTQ-2D) has no native code: its GPU path is
 * Triton kernels launched from Python, and each entry point names the reference function or
 * kernel whose work it takes over.
 */
#ifndef GPTQ2D_H
#define GPTQ2D_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GPTQ2D_EINVAL (-1)
#define GPTQ2D_EUNSUPPORTED (-2)
#define GPTQ2D_ESCRATCH (-3) /* the problem does not fit the fixed scratch of a *_noalloc entry point */

#define GPTQ2D_DECLARE(T, SUF)                                                                                        \
  /* Whole sweep with a built-in per-entry quantizer fused in: replaces the stage loop of              \
   * _gptq_2d_blocked (gptq_2d.py:1295-1375) with its _push/_flush_block launches                     \
   * (gptq_2d.py:244-378, 633-1119) and the quantizer plug-in calls (gptq_2d.py:147-164).             \
   * qkind 0: round half to even (quantizer_int.py:18-25); 1: affine with full-matrix scale qa and     \
   * zero point qb (quantizer_int.py:63-83, 161-244); 2: prescribed values qa (teacher forcing; no     \
   * reference counterpart).  ypre (optional, [B,m,n]) receives Y of every entry just before it is    \
   * rounded.  c, e: [B,m,n] scratch.  Stages of tiles [stage_begin, stage_end) (-1: to the end),     \
   * outer_tiles tile stages per outer block; both ends on outer-block boundaries (or stage_end at   \
   * the end of the sweep), else GPTQ2D_EINVAL; a later call resumes from the same y, c, e.  y is    \
   * updated in place.  m or n of 2^26 or more: GPTQ2D_EUNSUPPORTED (32-bit offsets inside a tile). */ \
  int gptq2d_sweep_fused_##SUF(T* y, T* c, T* e, const T* l, const T* u, int64_t m, int64_t n, int32_t bnd,         \
                               const int64_t* bshape, const int64_t* l_stride, const int64_t* u_stride,             \
                               int32_t qkind, const T* qa, const int64_t* qa_stride, const T* qb,                   \
                               const int64_t* qb_stride, double qmin, double qmax, T* ypre, int64_t outer_tiles,    \
                               int64_t stage_begin, int64_t stage_end, void* stream);                               \
  /* The fused sweep over p x q super-entries (gptq_2d_super_entry, gptq_2d.py:1421-1447, with a       \
   * built-in quantizer): p = q = 1 is gptq2d_sweep_fused; p = 1, q = 32 (one super-entry per tile     \
   * row, n % 32 == 0) sweeps each tile row by row, U's 32 x 32 diagonal blocks never read, with qkind \
   * 0-2 as above per entry or 3: the abs-max INT quantizer of each super-entry row from its current     \
   * values with the scale rounded to bf16 (dtype16 1) or fp16 (2) (int_abs_max_quantizer,              \
   * quantizer_int.py:120-134, 408-470); other shapes GPTQ2D_EUNSUPPORTED.  scale_out (optional,         \
   * [B,m,n], qkind 3 only): every entry receives the scale its row was rounded with (no reference       \
   * counterpart: the scales of a packed layer).  Other arguments as above. */                          \
  int gptq2d_sweep_fused_se_##SUF(T* y, T* c, T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t p,         \
                                  int64_t q, int32_t bnd, const int64_t* bshape, const int64_t* l_stride,           \
                                  const int64_t* u_stride, int32_t qkind, const T* qa, const int64_t* qa_stride,    \
                                  const T* qb, const int64_t* qb_stride, double qmin, double qmax, int32_t dtype16, \
                                  T* ypre, T* scale_out, int64_t outer_tiles, int64_t stage_begin,                  \
                                  int64_t stage_end, void* stream);                                                  \
  /* Tile edge of the fused sweep. */                                                                  \
  int64_t gptq2d_sweep_fused_tile_##SUF(void);                                                                       \
  /* The whole fused sweep (as gptq2d_sweep_fused with stage_begin 0, stage_end -1) with no c and e:     \
   * its scratch is a fixed device array of the library (128 MiB on every GPU that loads it, held until \
   * the process ends), so the call allocates nothing at all -- for callers that cannot allocate device  \
   * memory (code under stream capture, serving loops, allocation-free harnesses).  No counterpart in    \
   * the reference, which allocates its scratch per call from torch's caching allocator                 \
   * (gptq_2d.py:1324-1334).  B m n must not exceed gptq2d_sweep_fused_noalloc_capacity(sizeof(T)),     \
   * else GPTQ2D_ESCRATCH and nothing runs.  All calls on one GPU share its array: calls that overlap   \
   * on one GPU (other streams, other host threads) race and give wrong results. */                      \
  int gptq2d_sweep_fused_noalloc_##SUF(T* y, const T* l, const T* u, int64_t m, int64_t n, int32_t bnd,              \
                                       const int64_t* bshape, const int64_t* l_stride, const int64_t* u_stride,     \
                                       int32_t qkind, const T* qa, const int64_t* qa_stride, const T* qb,           \
                                       const int64_t* qb_stride, double qmin, double qmax, T* ypre,                 \
                                       int64_t outer_tiles, void* stream);                                           \
                                                                                                                      \
  /* Plug-in path, plain entries: push of stage s inside the block ending at s1 -- error, down and     \
   * right feedback, commit of z, capture of the next stage's values (_push_kernel,                   \
   * gptq_2d.py:244-378). */                                                                           \
  int gptq2d_push_plain_##SUF(T* y, T* c, T* e, const T* z, const T* old, T* next_old, const T* l, const T* u,     \
                              int64_t m, int64_t n, int64_t s, int64_t s1, int32_t bnd, const int64_t* bshape,    \
                              const int64_t* l_stride, const int64_t* u_stride, void* stream);                     \
  /* C += E at the sources of stages [s0, s1) (_add_own_errors_kernel, gptq_2d.py:382-425). */        \
  int gptq2d_add_own_errors_##SUF(T* c, const T* e, int64_t B, int64_t m, int64_t n, int64_t s0, int64_t s1,        \
                                  void* stream);                                                                    \
  /* Super-entry p x q push down through L (_push_down_super_entry_kernel, gptq_2d.py:429-533). */     \
  int gptq2d_push_down_se_##SUF(T* y, T* c, T* e, const T* z, const T* l, int64_t m, int64_t n, int64_t p,          \
                                int64_t q, int64_t s, int64_t s1, int32_t bnd, const int64_t* bshape,               \
                                const int64_t* l_stride, void* stream);                                             \
  /* Super-entry commit and push right through U (_push_right_super_entry_kernel,                     \
   * gptq_2d.py:537-629). */                                                                           \
  int gptq2d_push_right_se_##SUF(T* y, const T* c, const T* z, const T* u, int64_t m, int64_t n, int64_t p,         \
                                 int64_t q, int64_t s, int64_t s1, int32_t bnd, const int64_t* bshape,              \
                                 const int64_t* u_stride, void* stream);                                            \
  /* out[b, k] = Y[b] on antidiagonal s (the old-value copy of _gptq_2d_blocked, gptq_2d.py:1345-1348). */ \
  int gptq2d_gather_antidiagonal_##SUF(const T* y, T* out, int64_t B, int64_t m, int64_t n, int64_t s,             \
                                       void* stream);                                                               \
  /* x[0:count] = v (the zero-initialised C of gptq_2d.py:1324). */                                    \
  int gptq2d_fill_##SUF(T* x, double v, int64_t count, void* stream);                                                \
  /* Block flush: the errors of stages [s0, s1) into the targets s1 <= i/p + j/q < s_end, C += L E and \
   * Y += L E + C U over the band (_repack_errors + _flush_down + _flush_right, gptq_2d.py:633-1119). */ \
  int gptq2d_flush_##SUF(T* y, T* c, const T* e, const T* l, const T* u, int64_t m, int64_t n, int64_t p,           \
                         int64_t q, int64_t s0, int64_t s1, int64_t s_end, int32_t bnd, const int64_t* bshape,      \
                         const int64_t* l_stride, const int64_t* u_stride, void* stream);                           \
                                                                                                                      \
  /* Affine quantizer on the flat strided slice start + k*step, k < len, of each [msize] matrix        \
   * (_affine_quantize_kernel, quantizer_int.py:161-244). */                                           \
  int gptq2d_affine_quantize_##SUF(T* out, const T* y, const T* scale, const T* zp, int64_t msize, int64_t start,    \
                                   int64_t step, int64_t len, int32_t bnd, const int64_t* bshape,                   \
                                   const int64_t* scale_stride, const int64_t* zp_stride, double qmin, double qmax, \
                                   void* stream);                                                                   \
  /* Round half to even on the slice (round_quantizer, quantizer_int.py:18-25). */                    \
  int gptq2d_round_quantize_##SUF(T* out, const T* y, int64_t msize, int64_t start, int64_t step, int64_t len,     \
                                  int32_t bnd, const int64_t* bshape, void* stream);                               \
  /* Affine quantizer on a strided [d, p, q] super-entry view (_affine_quantize_super_entry_kernel,    \
   * quantizer_int.py:248-351). */                                                                     \
  int gptq2d_affine_quantize_se_##SUF(T* out, const T* y, const T* scale, const T* zp, int64_t msize, int64_t d,    \
                                      int64_t p, int64_t q, int64_t sd, int64_t sp, int64_t sq, int32_t bnd,        \
                                      const int64_t* bshape, const int64_t* scale_stride, const int64_t* zp_stride, \
                                      double qmin, double qmax, void* stream);                                      \
  /* Round half to even on a super-entry view (round_quantizer_super_entry, quantizer_int.py:28-35). */ \
  int gptq2d_round_quantize_se_##SUF(T* out, const T* y, int64_t msize, int64_t d, int64_t p, int64_t q, int64_t sd, \
                                     int64_t sp, int64_t sq, int32_t bnd, const int64_t* bshape, void* stream);     \
  /* Symmetric abs-max scale per row, rounded to bf16 (dtype16 1) or fp16 (2), zero -> 1            \
   * (_int_abs_max_scale_kernel, quantizer_int.py:354-404). */                                         \
  int gptq2d_absmax_scale_##SUF(T* out, const T* x, int64_t rows, int64_t size, int64_t row_stride,                 \
                                int64_t col_stride, double qmin, double qmax, int32_t dtype16, void* stream);       \
  /* Abs-max INT quantizer per row of each super-entry from its current values                        \
   * (_int_abs_max_quantize_kernel, quantizer_int.py:408-470).  scale_out (optional): a map laid out     \
   * like y (same view strides, matrices msize apart) whose entries receive their row's scale. */      \
  int gptq2d_absmax_quantize_se_##SUF(T* out, const T* y, int64_t msize, int64_t B, int64_t d, int64_t p, int64_t q, \
                                      int64_t sd, int64_t sp, int64_t sq, double qmin, double qmax, int32_t dtype16, \
                                      T* scale_out, void* stream);                                                  \
                                                                                                                      \
  /* Unit lower (block) triangular L with M^{-1} = L Lambda L^T for `batch` contiguous k x k SPD      \
   * matrices m; work: [batch, k, k] scratch; info[batch]: first non-positive pivot (1-based) or 0     \
   * (ldl_of_inverse, gptq_2d_reference.py:29-49).  size <= 128 (f32) or 64 (f64).  fp32 matrices with \
   * k % 4 == 0 are factored in groups of up to 16 that share every Cholesky launch; results equal    \
   * one call per matrix bit for bit. */                                                               \
  int gptq2d_ldl_of_inverse_##SUF(const T* m, T* out, T* work, int* info, int64_t batch, int64_t k, int64_t size,  \
                                  void* stream);                                                                    \
  /* ldl_of_inverse of one k x k matrix in parts, so that the Cholesky and the inverse of two          \
   * factorisations can be scheduled apart on two streams (the reference computes its factors one     \
   * after the other, demo.ipynb cell 5):                                                             \
   * col_begin == 0 starts (copies m into work); Cholesky panels of columns [col_begin, col_end)        \
   * (multiples of 64 for f32, 32 for f64; col_end < 0: to k); finish != 0: the inverse and the        \
   * normalisation into out.  One call with col_begin = 0, col_end = -1, finish = 1 equals             \
   * gptq2d_ldl_of_inverse with batch 1.  info[0] as there. */                                          \
  int gptq2d_ldl_of_inverse_part_##SUF(const T* m, T* out, T* work, int* info, int64_t k, int64_t size,            \
                                       int64_t col_begin, int64_t col_end, int32_t finish, void* stream);          \
  /* ldl_of_inverse of two matrices at once (the Kronecker factors of one layer; no reference         \
   * counterpart -- the reference computes them one after the other, demo.ipynb cell 5): matrix f      \
   * (m_f, k_f x k_f, block size size_f, outputs out_f, scratch work_f, info_f as above) on stream_f,   \
   * the first parts of the triangular inverses beside the factorisations (three distinct streams of  \
   * one device).  Two fp32 matrices of one size share every Cholesky launch; other pairs are         \
   * enqueued panel by panel, alternating.  The inverse of a factor's leading block starts as soon as \
   * its factorisation has passed it, and the normalisations wait for it.  Results equal two          \
   * gptq2d_ldl_of_inverse calls bit for bit; with upper1 != 0 (size1 == 1 only) out1 receives the     \
   * transpose of the second factor (U = L^T, the sweep's upper factor) written directly. */         \
  int gptq2d_ldl_of_inverse_pair_##SUF(const T* m0, T* out0, T* work0, int* info0, int64_t k0, int64_t size0,      \
                                       const T* m1, T* out1, T* work1, int* info1, int64_t k1, int64_t size1,      \
                                       int32_t upper1, void* stream0, void* stream1, void* stream2);               \
  /* Unit lower (block) triangular L with M = L Lambda L^T (ldl, gptq_2d_reference.py:52-55). */       \
  int gptq2d_ldl_##SUF(const T* m, T* out, T* work, int* info, int64_t batch, int64_t k, int64_t size,              \
                       void* stream);                                                                               \
  /* Strided batched GEMM D = beta D + alpha A B with triangular operand structure (tri: 0 dense,      \
   * 1 lower, 2 upper) -- the building block of the LDL; exported for tests.  No reference            \
   * counterpart (torch.linalg inside the reference's ldl_of_inverse). */                             \
  int gptq2d_gemm_##SUF(int64_t M, int64_t N, int64_t K, int64_t batch, const T* A, int64_t a_rs, int64_t a_cs,     \
                        int64_t a_bs, const T* B, int64_t b_rs, int64_t b_cs, int64_t b_bs, T* D, int64_t d_rs,      \
                        int64_t d_cs, int64_t d_bs, double alpha, double beta, int32_t a_tri, int32_t b_tri,        \
                        int32_t d_tri, void* stream);                                                               \
                                                                                                                      \
  /* Trellis (Viterbi) quantizer of `rows` contiguous sequences x[rows, steps*V] over the code table   \
   * table[2^L, V] (row s = the values of state s): the state path of least squared distance whose    \
   * consecutive states overlap in L - K*V bits (next = ((s << K*V) | h) mod 2^L), first-index ties,   \
   * with tail_biting != 0 the path circular (the reference's two-pass search on x rolled by half).    \
   * Replaces _viterbi_step_kernel / _viterbi_final_kernel / _viterbi_backtrack_kernel and their       \
   * driver _trellis_quantize_triton (quantizer_trellis.py:146-341) in one launch; the same search as   \
   * _viterbi / _trellis_quantize_torch (quantizer_trellis.py:82-143).  hist: caller-owned workspace of \
   * gptq2d_viterbi_workspace(rows, steps, L, K, V) elements (T), overwritten.  scale (optional,       \
   * [rows]): out = table values * scale.  out (optional, [rows, steps*V]) and states (optional,      \
   * [rows, steps], int64) receive the result.  1 <= L <= 24, V in {1, 2}, K*V <= min(L, 8). */      \
  int gptq2d_viterbi_##SUF(const T* x, const T* table, T* hist, const T* scale, T* out, int64_t* states,            \
                           int64_t rows, int64_t steps, int32_t L, int32_t K, int32_t V, int32_t tail_biting,      \
                           void* stream);                                                                           \
                                                                                                                      \
  /* Packed INT codes (no reference counterpart: the reference returns dequantized values only).  z     \
   * [B,m,n] holds affine-quantizer outputs (q - zp) * s, q integer in [qmin, qmax]; scale / zp are     \
   * read at b*stride[0] + i*stride[1] + j*stride[2] (zp optional: 0).  Code u = q - qmin in `bits` bits  \
   * (gptq2d_int_code_bits), little-endian bit fields per row: code j at bits [j*bits, (j+1)*bits) of   \
   * the row, bit k in bit k%32 of word k/32; row_words >= ceil(n*bits/32) words per row, tail zero.    \
   * bad (optional, [B*m]): per row, the entries not equal to (q - zp) * s for q = rint(z/s + zp) in    \
   * range (packed as 0). */                                                                            \
  int gptq2d_pack_int_##SUF(const T* z, int64_t B, int64_t m, int64_t n, const T* scale,                            \
                            const int64_t* scale_stride, const T* zp, const int64_t* zp_stride, double qmin,       \
                            double qmax, int32_t bits, uint32_t* words, int64_t row_words, int32_t* bad,           \
                            void* stream);                                                                          \
  /* z = (u + qmin - zp) * scale from packed codes: the inverse of gptq2d_pack_int (exact for a row   \
   * with no bad entries; a zero's sign is not kept). */                                                \
  int gptq2d_unpack_int_##SUF(const uint32_t* words, int64_t B, int64_t m, int64_t n, int64_t row_words,             \
                              const T* scale, const int64_t* scale_stride, const T* zp,                             \
                              const int64_t* zp_stride, double qmin, int32_t bits, T* z, void* stream);             \
  /* Decode trellis streams (see gptq2d_trellis_pack): sequence r = the p x q block (b, I, J) of a      \
   * [B,m,n] layout read row by row (a plain [R, T] array: B 1, m R, n T, p 1, q T), state t = the     \
   * L-bit window at stream bit t*K*V.  values (optional, the [B,m,n] layout): entries t*V .. t*V+V-1   \
   * of each block = table[s_t, v] * scale[r * scale_stride] (scale optional: 1), the trellis           \
   * quantizer's values (quantizer_trellis.py:143, 344-391); states (optional, [seqs, p*q/V] int64). */ \
  int gptq2d_trellis_unpack_##SUF(const uint32_t* words, int64_t B, int64_t m, int64_t n, int64_t p, int64_t q,       \
                                  int64_t row_words, int32_t L, int32_t K, int32_t V, int32_t tail_biting,           \
                                  const T* table, const T* scale, int64_t scale_stride, T* values, int64_t* states,  \
                                  void* stream);

/* gptq2d_sweep_fused_se_f32 on one matrix (no batch) with U = P (x) Q given by its Kronecker factors
 * instead of its n^2 entries: up [np, np] and uq [nq, nq] row-major, n = np nq, every entry of both
 * read (the product's own zeros and diagonal included), and U[i, j] = up[i / nq, j / nq] * uq[i % nq,
 * j % nq] formed as one fp32 product per use -- the entries of torch.kron(up, uq), so the result is
 * bit for bit that of gptq2d_sweep_fused_se_f32 with the explicit product.  qa and qb are [m, n]
 * (contiguous); other arguments as gptq2d_sweep_fused_se_f32.  Replaces the explicit U that the
 * reference's Algorithm 4 never forms (gptq_2d_reference.py:270-294 reads only the per-mode factors;
 * the reference's GPU sweep, gptq_2d.py:1378-1447, takes the n x n U).  GPTQ2D_EUNSUPPORTED unless
 * nq % 16 == 0, m < 2^20, n < 2^20, m % 4 == n % 4 == 0 and y, c, e, l, uq are 16-byte aligned, all
 * checked before any device work. */
int gptq2d_sweep_fused_kron_f32(float* y, float* c, float* e, const float* l, const float* up, const float* uq,
                                int64_t m, int64_t np, int64_t nq, int64_t p, int64_t q, int32_t qkind,
                                const float* qa, const float* qb, double qmin, double qmax, int32_t dtype16,
                                float* ypre, float* scale_out, int64_t outer_tiles, int64_t stage_begin,
                                int64_t stage_end, void* stream);

/* Largest B m n (elements per matrix of the batch) gptq2d_sweep_fused_noalloc_* accepts for elements of
 * elem_bytes bytes (4 or 8; -1 otherwise): 2^24 for float, 2^23 for double.  No counterpart in the
 * reference (see gptq2d_sweep_fused_noalloc). */
int64_t gptq2d_sweep_fused_noalloc_capacity(int32_t elem_bytes);

/* gptq2d_viterbi_f32 for a table given as E entries of W of its rows: urows[E][W][V] and ridx[2^L / W] (int32)
 * with table[s + w 2^L / W] == urows[ridx[s]][w] bit for bit -- W = 1: the distinct rows; W = 2: the distinct
 * pairs of the rows of states s and s + 2^(L-1) (HYB: 512 look-up rows with both signs, in either order: 1024).  Where 1 <= E <= 1024,
 * 2 <= K*V <= 4, max(4, 2^(K*V)) <= 2^(L-K*V) <= 4096 and table and hist are 16-byte aligned (e.g. HYB L = 16,
 * K*V = 4), each step first evaluates the entries' costs and the states read theirs from LDS (the same values,
 * so the same search); other shapes run gptq2d_viterbi_f32.  Bit 16 of ridx[s] (the entry in bits 0-15) sends
 * state s's reads to a second copy of the step's costs, placed in other LDS banks, where the two copies fit
 * beside a second workgroup per CU; it is ignored otherwise, and never changes the result.  Other arguments
 * and the result as gptq2d_viterbi_f32 (quantizer_trellis.py:146-341, 82-143). */
int gptq2d_viterbi_rows_f32(const float* x, const float* table, const float* urows, const int32_t* ridx, int64_t E,
                            int32_t W, float* hist, const float* scale, float* out, int64_t* states, int64_t rows,
                            int64_t steps, int32_t L, int32_t K, int32_t V, int32_t tail_biting, void* stream);

/* Elements of the history workspace gptq2d_viterbi_* needs for `rows` sequences of `steps` steps (-1 if
 * the arguments are invalid).  Part of the trellis quantizer above (quantizer_trellis.py:146-341 keeps its
 * step minima in a torch-allocated [steps, rows, 2^L] buffer). */
int64_t gptq2d_viterbi_workspace(int64_t rows, int64_t steps, int32_t L, int32_t K, int32_t V);

/* Bits of a packed INT code for integer qmin <= qmax: ceil(log2(qmax - qmin + 1)), -1 beyond 16 or for
 * non-integer bounds.  Part of the packed format (no reference counterpart). */
int32_t gptq2d_int_code_bits(double qmin, double qmax);

/* Words of one trellis stream of `steps` states: ceil(steps*K*V / 32) with tail_biting, else
 * ceil((steps*K*V + L - K*V) / 32); -1 for invalid arguments. */
int64_t gptq2d_trellis_stream_words(int64_t steps, int32_t L, int32_t K, int32_t V, int32_t tail_biting);

/* Pack bitshift-trellis paths (quantizer_trellis.py:82-143, which returns the states; the reference's
 * docstring, quantizer_trellis.py:11-16, counts T*K bits per tail-biting sequence but keeps no stream) into
 * one MSB-first stream per sequence: the top K*V bits of every state in order (stream bit k = bit 31-k%32
 * of word k/32), plus the low L - K*V bits of the last state without tail-biting.  Sequences as in
 * gptq2d_trellis_unpack_*; state t of a sequence is its entry t*copies (copies = V: a per-entry state map
 * in which each state repeats over the V entries it emitted, every copy checked; 1: one entry per state).
 * bad (optional, [seqs]): states out of [0, 2^L), breaks of s_{t+1} >> KV == s_t mod 2^(L-KV) (and, with
 * tail_biting, between the last state and the first) and disagreeing copies.  L <= 30. */
int gptq2d_trellis_pack(const int64_t* states, int64_t B, int64_t m, int64_t n, int64_t p, int64_t q, int32_t copies,
                        int32_t L, int32_t K, int32_t V, int32_t tail_biting, uint32_t* words, int64_t row_words,
                        int32_t* bad, void* stream);

GPTQ2D_DECLARE(float, f32)
GPTQ2D_DECLARE(double, f64)

#undef GPTQ2D_DECLARE

/* Launch profiler (no reference counterpart; the reference times with host clocks, demo.ipynb:109-118).
 * While on, every launch of a profiled kernel class is bracketed with HIP events on its stream.
 * Process-global, not thread-safe, not for use under stream capture.
 * kind 0: cross-tile feedback panels (flush); 1: fused tile sweeps; 2: LDL GEMMs. */
int gptq2d_profile_start(int64_t capacity, uint32_t kinds); /* kinds: bit k enables class k */
int gptq2d_profile_read(int32_t kind, double* ms, double* work, int64_t* launches);
int gptq2d_profile_stop(void);

#ifdef __cplusplus
}
#endif

#endif /* GPTQ2D_H */
