// TopologyConfig::get_exclusive_cores on synthetic multi-GPU topologies.
//
// The reference splits each NUMA node's physical cores evenly between the
// GPUs on that node, in GPU order, as runs of consecutive CPU numbers
// (include/gfd/pcie_topology.h:41-60 of the reference).  This program builds
// TopologyConfig values by hand (no sysfs, no GPU) and checks, for each:
//   - on nodes numbered consecutively, the reference's own result
//     (base = cpu_start + index_on_node * cores_per_gpu, stride 1), restated
//     here from that header as the expected value;
//   - on every layout, that each GPU's cores are physical cores of its own
//     node, that GPUs on one node get disjoint shares of equal size
//     node_cores / gpus_on_node, and that the shares are in GPU order;
//   - edge cases: a share whose numbering has a gap is cut at the gap, an
//     unknown node (-1) counts as node 0, a gpu_id out of range and a node
//     with fewer cores than GPUs give zero cores.
// Prints PASSED and exits 0 on success.
#include <gfd/pcie_topology.h>

#include <cstdio>
#include <set>
#include <vector>

static int failures = 0;

#define EXPECT(cond, ...)                                   \
    do {                                                    \
        if (!(cond)) {                                      \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);              \
            std::fprintf(stderr, "\n");                     \
            failures++;                                     \
        }                                                   \
    } while (0)

// One node's description: its physical cores (one CPU number per core).
struct Node {
    std::vector<int> cores;
};

// A topology of GPUs placed on nodes; gpu_node[g] is GPU g's node (-1 allowed).
static gfd::TopologyConfig make_topology(const std::vector<Node>& nodes, const std::vector<int>& gpu_node) {
    gfd::TopologyConfig t;
    t.num_gpus = (int)gpu_node.size();
    t.total_numa_nodes = (int)nodes.size();
    t.gpus_per_numa.assign(nodes.size(), 0);
    for (int n : gpu_node) t.gpus_per_numa[(size_t)(n >= 0 ? n : 0)]++;
    t.physical_cores_per_numa = (int)nodes[0].cores.size();
    t.cpus_per_numa = t.physical_cores_per_numa;
    for (size_t g = 0; g < gpu_node.size(); g++) {
        gfd::GpuTopology gt;
        gt.gpu_id = (int)g;
        gt.numa_node = gpu_node[g];
        const Node& nd = nodes[(size_t)(gpu_node[g] >= 0 ? gpu_node[g] : 0)];
        gt.node_cores = nd.cores;
        gt.node_cpus = nd.cores;
        gt.num_physical_cores = (int)nd.cores.size();
        gt.cpu_start = nd.cores.empty() ? 0 : nd.cores.front();
        gt.cpu_end = nd.cores.empty() ? 0 : nd.cores.back();
        gt.total_numa_nodes = (int)nodes.size();
        t.gpus.push_back(gt);
    }
    return t;
}

static Node consecutive(int first, int count) {
    Node n;
    for (int i = 0; i < count; i++) n.cores.push_back(first + i);
    return n;
}

static Node strided(int first, int count, int step) {
    Node n;
    for (int i = 0; i < count; i++) n.cores.push_back(first + i * step);
    return n;
}

// The reference's partition for consecutively numbered nodes (its
// pcie_topology.h:41-60): cores_per_gpu = cores_per_node / gpus_on_node,
// base = cpu_start + index_on_node * cores_per_gpu, stride 1.
static void reference_rule(const gfd::TopologyConfig& t, int gpu, int& base, int& n, int& stride) {
    const gfd::GpuTopology& g = t.gpus[(size_t)gpu];
    const int node = g.numa_node;
    const int per = g.num_physical_cores / t.gpus_per_numa[(size_t)node];
    int idx = 0;
    for (int i = 0; i < gpu; i++)
        if (t.gpus[(size_t)i].numa_node == node) idx++;
    stride = 1;
    base = g.cpu_start + idx * per;
    n = per;
    if (base + n - 1 > g.cpu_end) n = g.cpu_end - base + 1;
}

// Shares are physical cores of the GPU's own node, disjoint within the node,
// of equal size, in GPU order.
static void check_partition(const char* name, const gfd::TopologyConfig& t) {
    std::vector<std::set<int>> used(t.gpus_per_numa.size());
    std::vector<int> last_base(t.gpus_per_numa.size(), -1);
    for (int g = 0; g < t.num_gpus; g++) {
        int base = -1, n = -1, stride = -1;
        t.get_exclusive_cores(g, base, n, stride);
        const gfd::GpuTopology& gt = t.gpus[(size_t)g];
        const int node = gt.numa_node >= 0 ? gt.numa_node : 0;
        const int want = (int)gt.node_cores.size() / t.gpus_per_numa[(size_t)node];
        EXPECT(n == want, "%s gpu %d: %d cores, want %d", name, g, n, want);
        EXPECT(stride >= 1, "%s gpu %d: stride %d", name, g, stride);
        EXPECT(base > last_base[(size_t)node], "%s gpu %d: base %d not after %d", name, g, base,
               last_base[(size_t)node]);
        last_base[(size_t)node] = base;
        const std::set<int> node_cores(gt.node_cores.begin(), gt.node_cores.end());
        for (int k = 0; k < n; k++) {
            const int c = base + k * stride;
            EXPECT(node_cores.count(c) == 1, "%s gpu %d: CPU %d is not a core of node %d", name, g, c, node);
            EXPECT(used[(size_t)node].insert(c).second, "%s gpu %d: CPU %d given twice", name, g, c);
        }
    }
}

int main() {
    // 8 GPUs on 2 nodes of 64 consecutively numbered cores (4 + 4).
    {
        const std::vector<Node> nodes = {consecutive(0, 64), consecutive(64, 64)};
        const gfd::TopologyConfig t = make_topology(nodes, {0, 0, 0, 0, 1, 1, 1, 1});
        check_partition("8gpu-2node", t);
        for (int g = 0; g < 8; g++) {
            int b = 0, n = 0, s = 0, rb = 0, rn = 0, rs = 0;
            t.get_exclusive_cores(g, b, n, s);
            reference_rule(t, g, rb, rn, rs);
            EXPECT(b == rb && n == rn && s == rs, "8gpu-2node gpu %d: (%d,%d,%d) reference (%d,%d,%d)", g, b, n,
                   s, rb, rn, rs);
        }
        int b = 0, n = 0, s = 0;
        t.get_exclusive_cores(5, b, n, s);
        EXPECT(b == 80 && n == 16 && s == 1, "8gpu-2node gpu 5: (%d,%d,%d)", b, n, s);
    }
    // GPUs interleaved between nodes (0,1,0,1,...) and a node shared by 3.
    {
        const std::vector<Node> nodes = {consecutive(0, 48), consecutive(48, 48)};
        const gfd::TopologyConfig t = make_topology(nodes, {0, 1, 0, 1, 0});
        check_partition("interleaved", t);
        for (int g = 0; g < 5; g++) {
            int b = 0, n = 0, s = 0, rb = 0, rn = 0, rs = 0;
            t.get_exclusive_cores(g, b, n, s);
            reference_rule(t, g, rb, rn, rs);
            EXPECT(b == rb && n == rn && s == rs, "interleaved gpu %d: (%d,%d,%d) reference (%d,%d,%d)", g, b, n,
                   s, rb, rn, rs);
        }
        int b = 0, n = 0, s = 0;
        t.get_exclusive_cores(4, b, n, s);  // third GPU of node 0: cores 32..47
        EXPECT(b == 32 && n == 16 && s == 1, "interleaved gpu 4: (%d,%d,%d)", b, n, s);
        t.get_exclusive_cores(3, b, n, s);  // second GPU of node 1: cores 72..95
        EXPECT(b == 72 && n == 24 && s == 1, "interleaved gpu 3: (%d,%d,%d)", b, n, s);
    }
    // Nodes whose cores are numbered every other CPU (node 0 even, node 1 odd):
    // the shares follow the node's numbering with stride 2.
    {
        const std::vector<Node> nodes = {strided(0, 32, 2), strided(1, 32, 2)};
        const gfd::TopologyConfig t = make_topology(nodes, {0, 0, 1, 1});
        check_partition("strided", t);
        int b = 0, n = 0, s = 0;
        t.get_exclusive_cores(1, b, n, s);
        EXPECT(b == 32 && n == 16 && s == 2, "strided gpu 1: (%d,%d,%d)", b, n, s);
        t.get_exclusive_cores(2, b, n, s);
        EXPECT(b == 1 && n == 16 && s == 2, "strided gpu 2: (%d,%d,%d)", b, n, s);
    }
    // A node whose core numbers have a gap inside one share (cores 0-7 and
    // 16-23): the share is cut at the gap rather than naming CPUs 8-15, which
    // are not the node's; with two GPUs each share is one run and whole.
    {
        Node gap = consecutive(0, 8);
        for (int c = 16; c < 24; c++) gap.cores.push_back(c);
        const gfd::TopologyConfig t = make_topology({gap}, {0});
        int b = 0, n = 0, s = 0;
        t.get_exclusive_cores(0, b, n, s);
        EXPECT(b == 0 && n == 8 && s == 1, "gap gpu 0: (%d,%d,%d)", b, n, s);
        const gfd::TopologyConfig t2 = make_topology({gap}, {0, 0});
        check_partition("gap-2gpu", t2);
        t2.get_exclusive_cores(1, b, n, s);
        EXPECT(b == 16 && n == 8 && s == 1, "gap gpu 1 of 2: (%d,%d,%d)", b, n, s);
    }
    // 3 GPUs on a node of 64 cores: 21 each, the last core unused.
    {
        const gfd::TopologyConfig t = make_topology({consecutive(0, 64)}, {0, 0, 0});
        check_partition("uneven", t);
        int b = 0, n = 0, s = 0;
        t.get_exclusive_cores(2, b, n, s);
        EXPECT(b == 42 && n == 21 && s == 1, "uneven gpu 2: (%d,%d,%d)", b, n, s);
    }
    // Unknown node (-1) counts as node 0; out-of-range ids and a node with
    // fewer cores than GPUs give no cores.
    {
        const gfd::TopologyConfig t = make_topology({consecutive(0, 16)}, {-1, -1});
        check_partition("unknown-node", t);
        int b = 0, n = 0, s = 0;
        t.get_exclusive_cores(1, b, n, s);
        EXPECT(b == 8 && n == 8 && s == 1, "unknown-node gpu 1: (%d,%d,%d)", b, n, s);
        b = n = s = 7;
        t.get_exclusive_cores(2, b, n, s);
        EXPECT(n == 0, "gpu_id out of range: %d cores", n);
        t.get_exclusive_cores(-1, b, n, s);
        EXPECT(n == 0, "negative gpu_id: %d cores", n);
        const gfd::TopologyConfig small = make_topology({consecutive(0, 2)}, {0, 0, 0});
        small.get_exclusive_cores(0, b, n, s);
        EXPECT(n == 0, "2 cores for 3 GPUs: %d cores", n);
    }
    // Each MI355X has its own copy engines: the channel count does not drop
    // with the number of GPUs on a node.
    {
        const gfd::TopologyConfig t = make_topology({consecutive(0, 64)}, {0});
        const int one = t.recommended_ce_channels(1);
        EXPECT(one >= 1, "channels for 1 GPU: %d", one);
        for (int k = 2; k <= 8; k++)
            EXPECT(t.recommended_ce_channels(k) == one, "channels for %d GPUs: %d", k,
                   t.recommended_ce_channels(k));
    }
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("PASSED\n");
    return 0;
}
