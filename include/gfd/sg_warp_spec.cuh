#pragma once
// The reference's include name for the wave64 SG wave-specialised framework and GFD_SG_WARP_SPEC_KERNEL
// (include/gfd/sg_warp_spec.cuh of the reference), so device code written against
// it compiles unchanged.  HIP sources only.
#include "gfd/sg_warp_spec.h"
