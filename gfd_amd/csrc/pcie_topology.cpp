// GPU -> NUMA discovery and CPU selection (declaration: include/gfd/pcie_topology.h).
#include "gfd/pcie_topology.h"

#include <sched.h>

#include <algorithm>
#include <cctype>
#include <fstream>
#include <set>
#include <sstream>

#include "gfd/hip_shim.h"

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
    return t;
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
