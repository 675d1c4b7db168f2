#pragma once
// The reference's include name for the wave64 wave-specialised tile framework and GFD_WARP_SPEC_KERNEL(_DB)
// (include/gfd/warp_spec.cuh of the reference), so device code written against
// it compiles unchanged.  HIP sources only.
#include "gfd/warp_spec.h"
