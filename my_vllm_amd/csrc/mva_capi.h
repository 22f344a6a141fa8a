// Host-side error plumbing shared by every C-ABI entry point.
//
// Entry points never throw across the ABI: they return 0 on success and a
// negative status otherwise, with a message retrievable by mva_last_error().
#pragma once

#include <hip/hip_runtime.h>

namespace mva {

// Records `msg` as the calling thread's last error; returns -1.
int set_error(const char* msg);

// Returns 0 if the most recent launch on this thread succeeded, else records
// "<what>: <hip error string>" and returns -2.
int check_launch(const char* what);

}  // namespace mva
