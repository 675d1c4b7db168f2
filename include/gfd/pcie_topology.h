#pragma once
// GPU -> NUMA node discovery and CPU selection for the poller and gather
// workers (the single-GPU part of include/gfd/pcie_topology.h:63-154 of the
// reference: PCI bus id -> /sys/bus/pci/devices/<bdf>/numa_node -> node
// cpulist).  CPU choice also honours the process affinity mask, so a job
// confined to a CPU share only pins threads to CPUs it may run on.
#include <string>
#include <vector>

namespace gfd {

struct GpuTopology {
    int gpu_id = 0;
    int numa_node = -1;          // -1 when the platform does not report one
    std::string pci_bus_id;      // "0000:xx:yy.z"
    std::vector<int> node_cpus;  // CPUs of numa_node, ascending (all CPUs if unknown)
    int total_numa_nodes = 1;
};

// Query HIP for the device's PCI bus id and read sysfs.
GpuTopology discover_gpu_topology(int gpu_id);

// CPUs this process may run on (sched_getaffinity), ascending.
std::vector<int> allowed_cpus();

// CPUs in /sys/devices/system/node/node<N>/cpulist (empty if absent).
std::vector<int> numa_node_cpus(int node);

// Parse a sysfs CPU list such as "0-3,8,10-11".
std::vector<int> parse_cpu_list(const std::string& s);

// Choose up to `want` CPUs for gather threads.
//   exclusive_core_base >= 0 && exclusive_core_count > 0: the reference rule
//     (src/cpu_polling.cpp:247-283): stride 2 when >= 16 cores, else 1,
//     CPUs base, base+stride, ...; CPUs outside the affinity mask are dropped.
//   otherwise: allowed CPUs on the GPU's node first, then other allowed CPUs,
//     one hyperthread per physical core before siblings.
std::vector<int> pick_cpus(const GpuTopology& topo, int want, int exclusive_core_base,
                           int exclusive_core_count);

}  // namespace gfd
