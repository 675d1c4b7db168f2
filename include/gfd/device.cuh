#pragma once
// The reference's include name for the wave64 device submit / commit / wait API
// (include/gfd/device.cuh of the reference), so device code written against
// it compiles unchanged.  HIP sources only.
#include "gfd/device.h"
