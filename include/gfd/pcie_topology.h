#pragma once
// GPU -> NUMA node discovery and CPU selection for the poller and gather
// workers (include/gfd/pcie_topology.h of the reference).
//
// The reference's names and fields are kept (GpuTopology, TopologyConfig,
// discover_topology, print_topology, recommended_ce_channels,
// get_exclusive_cores: pcie_topology.h:16-172), so callers written against
// them compile.  Values come from sysfs: the GPU's PCI bus id (from HIP) ->
// /sys/bus/pci/devices/<bdf>/numa_node -> the node's cpulist, and each CPU's
// thread_siblings_list for cores and hyperthreads.  The reference assumes
// every node is one contiguous CPU range of the same size plus one sibling
// range; here each node's own list is read.  CPU choice for the gather
// threads also honours the process affinity mask, so a job confined to a CPU
// share only pins threads to CPUs it may run on.
#include <string>
#include <vector>

namespace gfd {

struct GpuTopology {
    int gpu_id = 0;
    int numa_node = -1;          // -1 when the platform does not report one
    int pcie_bus = 0;            // PCI bus number of the GPU
    int cpu_start = 0;           // lowest physical core of the node
    int cpu_end = 0;             // highest physical core of the node
    int ht_offset = 0;           // second hyperthread of core c is c + ht_offset (0: no SMT)
    int num_physical_cores = 0;  // physical cores of the node
    // Not in the reference:
    std::string pci_bus_id;      // "0000:xx:yy.z"
    std::vector<int> node_cpus;  // CPUs of numa_node, ascending (all CPUs if unknown)
    std::vector<int> node_cores; // one CPU per physical core of the node, ascending
    int total_numa_nodes = 1;
};

struct TopologyConfig {
    int num_gpus = 0;
    int total_numa_nodes = 1;
    int cpus_per_numa = 0;            // logical CPUs of node 0 (or of the first GPU's node)
    int physical_cores_per_numa = 0;  // physical cores of that node
    std::vector<GpuTopology> gpus;
    std::vector<int> gpus_per_numa;

    // Copy channels per GPU.  Each MI355X has its own SDMA engines and its own
    // x16 link, so GPUs sharing a node do not share engines: the default
    // channel count holds whatever the sharing (the reference returns 3/2/1
    // for its shared copy engines, pcie_topology.h:35-39).
    int recommended_ce_channels(int active_gpus_on_same_numa) const;

    // This GPU's share of its node's physical cores: the node's cores split
    // evenly between the GPUs on that node, in GPU order (the reference's
    // partition rule, pcie_topology.h:41-60), as CPUs base, base + stride,
    // ..., base + (num - 1) * stride.  stride is 1 on nodes numbered
    // consecutively (the reference's only case); a share whose numbering has
    // a gap is cut at the gap.  num is 0 for an unknown gpu_id or a node with
    // fewer cores than GPUs.
    void get_exclusive_cores(int gpu_id, int& out_base_cpu, int& out_num_cores, int& out_stride) const;
};

// Topology of GPUs 0 .. num_gpus-1 (reference pcie_topology.h:63-154).
TopologyConfig discover_topology(int num_gpus);

// Log the topology at info level (reference pcie_topology.h:156-172).
void print_topology(const TopologyConfig& topo);

// One GPU: query HIP for the device's PCI bus id and read sysfs.
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
