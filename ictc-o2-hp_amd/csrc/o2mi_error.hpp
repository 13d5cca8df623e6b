// Shared state of the C ABI translation units: the per-thread status text
// (o2mi_last_error) and the optional kernel timing (o2mi_kernel_timing).
#pragma once

#include <hip/hip_runtime.h>

#include <string>

std::string& o2mi_error_slot();

// Kinds of timed launches (index of o2mi_kernel_timing_read_kinds).
enum {
  O2MI_TIMED_TP_FORWARD = 0,
  O2MI_TIMED_TP_BACKWARD = 1,
  O2MI_TIMED_RADIAL_FORWARD = 2,
  O2MI_TIMED_RADIAL_BACKWARD = 3,
  O2MI_TIMED_RADIAL_WEIGHT = 4,
  O2MI_TIMED_UVU_FORWARD = 5,   // the per-row-weight uvu kernels
  O2MI_TIMED_UVU_BACKWARD = 6,
  O2MI_TIMED_KINDS = 7,
};

struct O2miTimed {
  int kind;
  hipEvent_t start, stop;
};

// Records the start event when timing is enabled (returns false otherwise).
bool o2mi_timing_begin(hipStream_t s, O2miTimed* launch, int kind);
void o2mi_timing_end(hipStream_t s, O2miTimed* launch);
