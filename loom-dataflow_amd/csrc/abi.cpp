// abi.cpp -- library-wide C ABI entry points (version string).
//
// The kernels' entry points live next to their kernels (gemm.hip,
// attention.hip, decode.hip, mamba.hip); this file holds what belongs to the
// library as a whole.  The version string is the counterpart of the
// reference pybind module's __version__ (lib/pipeline/src/loom_pybind.cpp:19).
#include "../../include/loom_hip.h"

#define LOOM_HIP_VERSION_STRING "loom_hip 0.1.0 gfx950"

extern "C" const char* loom_hip_version(void) { return LOOM_HIP_VERSION_STRING; }
