// Library identification string.
#include "jinf/kernels_ext.h"

extern "C" const char* jinf_hip_version(void) { return "jinf_hip 0.1.0 gfx950"; }
