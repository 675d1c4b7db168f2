// GPU -> NUMA discovery and CPU selection (declaration: include/gfd/pcie_topology.h).
#include "gfd/pcie_topology.h"

#include <sched.h>

#include <algorithm>
#include <cctype>
#include <fstream>
#include <set>
#include <sstream>
#include <cstdio>

#include "gfd/copy_engine.h"
#include "gfd/hip_shim.h"
#include "gfd/log.h"

namespace gfd {

namespace {

std::string read_line(const std::string& path) {
    std::ifstream f(path);
    std::string s;
    if (f) std::getline(f, s);
    return s;
}

// First sibling listed for the CPU's core (identifies the physical core).
int core_key(int cpu) {
    auto v = parse_cpu_list(
        read_line("/sys/devices/system/cpu/cpu" + std::to_string(cpu) + "/topology/thread_siblings_list"));
    return v.empty() ? cpu : v.front();
}

}  // namespace

std::vector<int> parse_cpu_list(const std::string& s) {
    std::vector<int> out;
    std::stringstream ss(s);
    std::string tok;
    while (std::getline(ss, tok, ',')) {
        tok.erase(std::remove_if(tok.begin(), tok.end(), [](unsigned char c) { return std::isspace(c); }),
                  tok.end());
        if (tok.empty()) continue;
        size_t dash = tok.find('-');
        try {
            if (dash == std::string::npos) {
                out.push_back(std::stoi(tok));
            } else {
                int a = std::stoi(tok.substr(0, dash)), b = std::stoi(tok.substr(dash + 1));
                for (int c = a; c <= b; c++) out.push_back(c);
            }
        } catch (...) {
        }
    }
    std::sort(out.begin(), out.end());
    out.erase(std::unique(out.begin(), out.end()), out.end());
    return out;
}

std::vector<int> allowed_cpus() {
    std::vector<int> out;
    cpu_set_t cs;
    CPU_ZERO(&cs);
    if (sched_getaffinity(0, sizeof(cs), &cs) == 0)
        for (int c = 0; c < CPU_SETSIZE; c++)
            if (CPU_ISSET(c, &cs)) out.push_back(c);
    return out;
}

std::vector<int> numa_node_cpus(int node) {
    if (node < 0) return {};
    return parse_cpu_list(read_line("/sys/devices/system/node/node" + std::to_string(node) + "/cpulist"));
}

GpuTopology discover_gpu_topology(int gpu_id) {
    GpuTopology t;
    t.gpu_id = gpu_id;
    char bus[64] = {0};
    if (gfd_hip_pci_bus_id(bus, sizeof(bus), gpu_id) == 0) {
        std::string b(bus);
        for (auto& ch : b) ch = (char)std::tolower((unsigned char)ch);
        t.pci_bus_id = b;
        unsigned dom = 0, busno = 0, dev = 0, fn = 0;
        if (std::sscanf(b.c_str(), "%x:%x:%x.%x", &dom, &busno, &dev, &fn) == 4) t.pcie_bus = (int)busno;
        std::string n = read_line("/sys/bus/pci/devices/" + b + "/numa_node");
        if (!n.empty()) {
            try {
                t.numa_node = std::stoi(n);
            } catch (...) {
                t.numa_node = -1;
            }
        }
    }
    auto online = parse_cpu_list(read_line("/sys/devices/system/node/online"));
    t.total_numa_nodes = online.empty() ? 1 : (int)online.size();
    t.node_cpus = numa_node_cpus(t.numa_node);
    if (t.node_cpus.empty()) t.node_cpus = allowed_cpus();
    // Physical cores: the CPUs that are the first of their sibling list.
    std::set<int> seen;
    for (int c : t.node_cpus)
        if (seen.insert(core_key(c)).second) t.node_cores.push_back(c);
    t.num_physical_cores = (int)t.node_cores.size();
    if (!t.node_cores.empty()) {
        t.cpu_start = t.node_cores.front();
        t.cpu_end = t.node_cores.back();
        const auto sib = parse_cpu_list(read_line("/sys/devices/system/cpu/cpu" + std::to_string(t.cpu_start) +
                                                  "/topology/thread_siblings_list"));
        t.ht_offset = sib.size() > 1 ? sib[1] - sib[0] : 0;
    }
    return t;
}

TopologyConfig discover_topology(int num_gpus) {
    TopologyConfig topo;
    topo.num_gpus = num_gpus > 0 ? num_gpus : 0;
    for (int g = 0; g < topo.num_gpus; g++) topo.gpus.push_back(discover_gpu_topology(g));
    auto online = parse_cpu_list(read_line("/sys/devices/system/node/online"));
    const int max_node = online.empty() ? 0 : online.back();
    topo.total_numa_nodes = max_node + 1;
    // Node sizes: those of the first GPU's node, else of node 0.
    int node = topo.gpus.empty() || topo.gpus[0].numa_node < 0 ? 0 : topo.gpus[0].numa_node;
    std::vector<int> cpus = numa_node_cpus(node);
    if (cpus.empty()) cpus = allowed_cpus();
    std::set<int> cores;
    for (int c : cpus) cores.insert(core_key(c));
    topo.cpus_per_numa = (int)cpus.size();
    topo.physical_cores_per_numa = (int)cores.size();
    topo.gpus_per_numa.assign((size_t)topo.total_numa_nodes, 0);
    for (auto& g : topo.gpus) {
        // A GPU whose node is unknown counts against node 0, as in the reference's fallback.
        const int n = g.numa_node >= 0 && g.numa_node < topo.total_numa_nodes ? g.numa_node : 0;
        topo.gpus_per_numa[(size_t)n]++;
    }
    return topo;
}

int TopologyConfig::recommended_ce_channels(int active_gpus_on_same_numa) const {
    (void)active_gpus_on_same_numa;
    return DEFAULT_CE_CHANNELS;
}

void TopologyConfig::get_exclusive_cores(int gpu_id, int& out_base_cpu, int& out_num_cores, int& out_stride) const {
    out_base_cpu = 0;
    out_num_cores = 0;
    out_stride = 1;
    if (gpu_id < 0 || gpu_id >= (int)gpus.size()) return;
    const GpuTopology& g = gpus[(size_t)gpu_id];
    const int node = g.numa_node >= 0 && g.numa_node < (int)gpus_per_numa.size() ? g.numa_node : 0;
    const int sharing = gpus_per_numa.empty() ? 1 : std::max(1, gpus_per_numa[(size_t)node]);
    int idx = 0;  // GPUs before this one on the same node
    for (int i = 0; i < gpu_id; i++) {
        const int n = gpus[(size_t)i].numa_node >= 0 ? gpus[(size_t)i].numa_node : 0;
        if (n == node) idx++;
    }
    const int per = (int)g.node_cores.size() / sharing;
    if (per <= 0) return;
    // The share is a run of `per` of the node's physical cores in ascending
    // order, reported as base, base + stride, ..., base + (num - 1) * stride:
    // stride is the spacing of the share's first two cores (1 on a node whose
    // cores are numbered consecutively).  Where the numbering inside the share
    // is not evenly spaced, num stops at the first core off that progression,
    // so the triple never names a CPU outside the share.
    const size_t first = (size_t)(idx * per);
    out_base_cpu = g.node_cores[first];
    out_num_cores = 1;
    if (per > 1) {
        const int step = g.node_cores[first + 1] - g.node_cores[first];
        if (step <= 0) return;
        while (out_num_cores < per &&
               g.node_cores[first + (size_t)out_num_cores] == out_base_cpu + out_num_cores * step)
            out_num_cores++;
        out_stride = step;
    }
}

void print_topology(const TopologyConfig& topo) {
    GFD_LOG_INFO("Topology: %d GPU(s), %d NUMA node(s), %d physical cores per node\n", topo.num_gpus,
                 topo.total_numa_nodes, topo.physical_cores_per_numa);
    for (int g = 0; g < topo.num_gpus; g++) {
        int base = 0, n = 0, stride = 1;
        topo.get_exclusive_cores(g, base, n, stride);
        GFD_LOG_INFO("  GPU %d (%s): NUMA %d, cores %d-%d (stride %d, %d cores)\n", g,
                     topo.gpus[(size_t)g].pci_bus_id.c_str(), topo.gpus[(size_t)g].numa_node, base,
                     base + (n > 0 ? n - 1 : 0) * stride, stride, n);
    }
    for (int n = 0; n < topo.total_numa_nodes && n < (int)topo.gpus_per_numa.size(); n++)
        GFD_LOG_INFO("  NUMA %d: %d GPU(s), %d copy channel(s) per GPU\n", n, topo.gpus_per_numa[(size_t)n],
                     topo.recommended_ce_channels(topo.gpus_per_numa[(size_t)n]));
}

std::vector<int> pick_cpus(const GpuTopology& topo, int want, int exclusive_core_base,
                           int exclusive_core_count) {
    std::vector<int> allowed = allowed_cpus();
    std::set<int> allow(allowed.begin(), allowed.end());
    std::vector<int> out;
    if (want <= 0) return out;
    if (exclusive_core_base >= 0 && exclusive_core_count > 0) {
        int stride = exclusive_core_count >= 16 ? 2 : 1;
        for (int c = exclusive_core_base; c < exclusive_core_base + exclusive_core_count && (int)out.size() < want;
             c += stride)
            if (allow.count(c)) out.push_back(c);
        return out;
    }
    // Node CPUs first, then the rest; one hyperthread per core before siblings.
    std::vector<int> order;
    for (int c : topo.node_cpus)
        if (allow.count(c)) order.push_back(c);
    for (int c : allowed)
        if (std::find(order.begin(), order.end(), c) == order.end()) order.push_back(c);
    std::set<int> cores_used;
    std::vector<int> siblings;
    for (int c : order) {
        int k = core_key(c);
        if (cores_used.insert(k).second)
            out.push_back(c);
        else
            siblings.push_back(c);
        if ((int)out.size() >= want) return out;
    }
    for (int c : siblings) {
        out.push_back(c);
        if ((int)out.size() >= want) break;
    }
    return out;
}

}  // namespace gfd
