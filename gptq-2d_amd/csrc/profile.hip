// HIP-event launch profiler (see profile.h) and its C entry points.
#include "profile.h"

#include <vector>

#include "common.h"

namespace {

struct KindState {
  std::vector<hipEvent_t> start, stop;
  std::vector<double> work;
  int64_t used = 0;
};

struct Profiler {
  bool on = false;
  uint32_t mask = 0;
  KindState kind[PROF_KINDS];
};

Profiler g_prof;

void release() {
  for (auto& k : g_prof.kind) {
    for (auto e : k.start) (void)hipEventDestroy(e);
    for (auto e : k.stop) (void)hipEventDestroy(e);
    k.start.clear();
    k.stop.clear();
    k.work.clear();
    k.used = 0;
  }
  g_prof.on = false;
}

}  // namespace

bool gptq2d_prof_on(int32_t kind) {
  return g_prof.on && kind >= 0 && kind < PROF_KINDS && (g_prof.mask >> kind & 1u) &&
         g_prof.kind[kind].used < (int64_t)g_prof.kind[kind].start.size();
}

void gptq2d_prof_begin(int32_t kind, hipStream_t stream) {
  if (!gptq2d_prof_on(kind)) return;
  KindState& k = g_prof.kind[kind];
  (void)hipEventRecord(k.start[k.used], stream);
}

void gptq2d_prof_end(int32_t kind, double work, hipStream_t stream) {
  if (!gptq2d_prof_on(kind)) return;
  KindState& k = g_prof.kind[kind];
  (void)hipEventRecord(k.stop[k.used], stream);
  k.work[k.used] = work;
  ++k.used;
}

extern "C" {

// Turn profiling on for the kernel classes in `kinds` (bit k: class k) with room for `capacity`
// launches per class (creates the events).  Launches beyond the capacity are not recorded.
// Returns 0 or a hipError_t.
int gptq2d_profile_start(int64_t capacity, uint32_t kinds) {
  release();
  if (capacity <= 0) return GPTQ2D_EINVAL;
  g_prof.mask = kinds;
  for (int kind = 0; kind < PROF_KINDS; ++kind) {
    if (!(kinds >> kind & 1u)) continue;
    KindState& k = g_prof.kind[kind];
    k.start.resize(capacity);
    k.stop.resize(capacity);
    k.work.assign(capacity, 0.);
    for (int64_t i = 0; i < capacity; ++i) {
      int rc = (int)hipEventCreate(&k.start[i]);
      if (!rc) rc = (int)hipEventCreate(&k.stop[i]);
      if (rc) {
        k.start.resize(i);
        k.stop.resize(i);
        release();
        return rc;
      }
    }
  }
  g_prof.on = true;
  return 0;
}

// Totals of one kernel class since profile_start: summed launch time (ms, waits for the events),
// summed algorithmic work and the number of launches.
int gptq2d_profile_read(int32_t kind, double* ms, double* work, int64_t* launches) {
  if (kind < 0 || kind >= PROF_KINDS || !ms || !work || !launches) return GPTQ2D_EINVAL;
  KindState& k = g_prof.kind[kind];
  double t = 0., w = 0.;
  for (int64_t i = 0; i < k.used; ++i) {
    int rc = (int)hipEventSynchronize(k.stop[i]);
    if (rc) return rc;
    float e = 0.f;
    rc = (int)hipEventElapsedTime(&e, k.start[i], k.stop[i]);
    if (rc) return rc;
    t += e;
    w += k.work[i];
  }
  *ms = t;
  *work = w;
  *launches = k.used;
  return 0;
}

// Turn profiling off and free the events.
int gptq2d_profile_stop(void) {
  release();
  return 0;
}

}  // extern "C"
