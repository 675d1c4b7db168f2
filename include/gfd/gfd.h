#pragma once
// GFD host API in one include: the header every reference caller starts with
// (include/gfd/gfd.h:23-30 of the reference), with the same set of host
// components.  Host code only; it compiles with any C++17 compiler (no HIP
// headers are pulled in).
//
// Device code includes the wave64 device API by the reference's names:
//   <gfd/device.cuh>                submit / commit / wait (device.h)
//   <gfd/device_primitives.cuh>     tile and chunk primitives (device_primitives.h)
//   <gfd/warp_spec.cuh>             GFD_WARP_SPEC_KERNEL(_DB) (warp_spec.h)
//   <gfd/sg_device_primitives.cuh>  sg:: list primitives (sg_device_primitives.h)
//   <gfd/sg_warp_spec.cuh>          GFD_SG_WARP_SPEC_KERNEL (sg_warp_spec.h)
#include "gfd/descriptor_queue.h"
#include "gfd/tiled_queue.h"
#include "gfd/sg_task_queue.h"
#include "gfd/copy_engine.h"
#include "gfd/cpu_polling.h"
#include "gfd/warp_spec_session.h"
#include "gfd/staging_pool.h"
#include "gfd/pcie_topology.h"
