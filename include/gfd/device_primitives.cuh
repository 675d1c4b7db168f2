#pragma once
// The reference's include name for the wave64 tile and chunk primitives of the tiled queue
// (include/gfd/device_primitives.cuh of the reference), so device code written against
// it compiles unchanged.  HIP sources only.
#include "gfd/device_primitives.h"
