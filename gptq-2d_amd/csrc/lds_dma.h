// Buffer-resource loads straight into LDS (gfx950), shared by the MFMA kernels that stage panels
// through LDS without passing them through registers.
#pragma once

#include "common.h"

namespace {

// Raw buffer resource over `elems` floats from `base`: loads at a byte offset at or beyond the
// extent return zeros without touching memory, stores there are dropped -- which is how masked
// staging loads and epilogue stores are made without branches.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t matrix_rsrc(const float* base, int64_t elems) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)(elems * 4), 0x00020000);
}
constexpr int OOB = 0x7ffffff0;  // a byte offset past every extent these kernels accept

// Swizzle of the 16-byte k-quads of a staged 32-float panel row: quad q of row `row` is stored at quad
// position q ^ quad_swizzle(row).  A 128-bit operand read has the lanes of 32 consecutive rows read one
// quad each; over row % 32, (r ^ (r >> 3)) % 8 gives distinct positions to any 8 consecutive rows (an LDS
// of 32 banks serves 8 such lanes a cycle) and to any 8 rows of one parity among 16 consecutive ones (an
// LDS of 64 banks serves 16 lanes a cycle, rows r and r + 1 lying 32 banks apart), so neither stalls on
// bank conflicts.  (The plain row % 8 puts rows r and r + 8 on one bank group of a 64-bank LDS: counters
// showed a conflict cycle for every MFMA of the flush.)
__device__ __forceinline__ int quad_swizzle(int row) {
  const int r = row & 31;
  return (r ^ (r >> 3)) & 7;
}

typedef __attribute__((address_space(3))) float lds_float;

// LDS-direct load of W floats per lane (W = 4: 128 bits, W = 1: 32 bits) from byte offset `off` of
// buffer r: lane l's data lands at dst + W l (dst uniform); an offset past the buffer writes zeros.
// M0 carries the LDS address (one wait state before the load) and is restored afterwards.  Written
// as assembly so that the compiler does not order the load before the LDS reads of the other
// buffer; the caller orders it with wait_dma() and a barrier.
template <int W>
__device__ __forceinline__ void dma_load(__amdgpu_buffer_rsrc_t r, float* dst, int off) {
  const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_float*)dst);
  unsigned saved;
  if constexpr (W == 4)
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(r), "s"(lds)
        : "memory");
  else
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dword %1, %2, 0 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(r), "s"(lds)
        : "memory");
}
// dma_load with a wave-uniform byte offset `soff` added in the instruction's scalar offset field, so that
// a loop can step through a matrix with a loop-invariant per-lane offset and no vector instruction.  Only
// for loads whose every lane is in range (the scalar offset is not part of the buffer's range check).
template <int W>
__device__ __forceinline__ void dma_load_so(__amdgpu_buffer_rsrc_t r, float* dst, int off, int soff) {
  const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(lds_float*)dst);
  unsigned saved;
  if constexpr (W == 4)
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(r), "s"(lds), "s"(soff)
        : "memory");
  else
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dword %1, %2, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(off), "s"(r), "s"(lds), "s"(soff)
        : "memory");
}
// All of this wave's LDS-direct loads have landed.
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

}  // namespace
