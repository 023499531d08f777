// Opt-in per-launch timing of the engine's kernels with HIP events, for the benchmark's roofline
// figures.  While profiling is on, the host loops bracket every launch of a profiled kernel class
// with two events on the launch stream and add that launch's algorithmic flop (or byte) count.
// Off by default; the state is process-global and not thread-safe (one profiled run at a time),
// and events must not be recorded under stream capture, so a capturing caller leaves it off.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

enum ProfKind : int32_t {
  PROF_FLUSH = 0,        // cross-tile feedback panels (fused engine)
  PROF_TILE_SWEEP = 1,   // in-tile antidiagonal sweeps (fused engine)
  PROF_LDL_GEMM = 2,     // GEMM-shaped parts of the LDL preprocessing
  PROF_KINDS = 3,
};

// True while profiling is on for this kind and there are events left.
bool gptq2d_prof_on(int32_t kind);
// Record the start event of one launch (call just before the launch).
void gptq2d_prof_begin(int32_t kind, hipStream_t stream);
// Record the end event and the launch's algorithmic work (call just after the launch).
void gptq2d_prof_end(int32_t kind, double work, hipStream_t stream);
