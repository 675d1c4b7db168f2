#pragma once
// The reference's include name for the wave64 sg:: list allocation, commit and wait primitives
// (include/gfd/sg_device_primitives.cuh of the reference), so device code written against
// it compiles unchanged.  HIP sources only.
#include "gfd/sg_device_primitives.h"
