// Host-side construction of the dense layer's processing order (no device code): the order in
// which the row backward walks the input rows.  Built whenever a layer's connections change
// (initialisation, rewiring), so it runs on the host in linear time.
//
// The graph has one vertex per input row and one edge (a, b) per connection run.  The order
// is the preorder of a depth-first spanning forest of that graph in which each vertex's
// children are visited in increasing order of their subtree sizes (ties: discovery order);
// vertices without edges come last, in index order.  Searches start from the highest-degree
// unvisited vertex (ties: lowest index) and scan a vertex's neighbours in edge order (its
// operand-a runs in run order, then its operand-b runs).  A subtree occupies consecutive
// positions, so an edge between a parent and its child spans only the child's smaller
// siblings' subtrees: the two rows of most runs are processed close together in time.
#include "common.h"

#include <algorithm>
#include <numeric>
#include <vector>

extern "C" int cl_plan_locality_order(const int32_t* ra, const int32_t* rb, int64_t num_runs,
                                      int64_t in_dim, int32_t* order) {
    cl::clear_error();
    CL_ARG(num_runs >= 0 && in_dim >= 0, "negative size");
    CL_ARG(in_dim < (int64_t(1) << 31) && num_runs < (int64_t(1) << 30), "graph too large");
    CL_ARG(in_dim == 0 || order, "null pointer argument");
    CL_ARG(num_runs == 0 || (ra && rb), "null pointer argument");
    const int n = int(in_dim);
    const int64_t m = num_runs;
    for (int64_t r = 0; r < m; ++r)
        CL_ARG(ra[r] >= 0 && ra[r] < n && rb[r] >= 0 && rb[r] < n,
               "run %lld has an input outside [0, %d)", (long long)r, n);
    // adjacency in edge order: for vertex u, first the b of runs with a == u, then the a of
    // runs with b == u (a counting sort of the sources, stable)
    std::vector<int64_t> ptr(size_t(n) + 1, 0);
    for (int64_t r = 0; r < m; ++r) {
        ++ptr[size_t(ra[r]) + 1];
        ++ptr[size_t(rb[r]) + 1];
    }
    for (int u = 0; u < n; ++u) ptr[size_t(u) + 1] += ptr[size_t(u)];
    std::vector<int32_t> nbr(size_t(2 * m));
    {
        std::vector<int64_t> fill(ptr.begin(), ptr.end() - 1);
        for (int64_t r = 0; r < m; ++r) nbr[size_t(fill[size_t(ra[r])]++)] = rb[r];
        for (int64_t r = 0; r < m; ++r) nbr[size_t(fill[size_t(rb[r])]++)] = ra[r];
    }
    std::vector<int32_t> seeds(static_cast<size_t>(n));
    std::iota(seeds.begin(), seeds.end(), 0);
    std::stable_sort(seeds.begin(), seeds.end(), [&](int32_t x, int32_t y) {
        return (ptr[size_t(x) + 1] - ptr[size_t(x)]) > (ptr[size_t(y) + 1] - ptr[size_t(y)]);
    });
    // depth-first spanning forest; children in discovery order
    constexpr int32_t kUnseen = -2, kRoot = -1;
    std::vector<int32_t> parent(size_t(n), kUnseen);
    std::vector<int32_t> child_first(size_t(n), -1), child_last(size_t(n), -1),
        child_next(size_t(n), -1);
    std::vector<int32_t> roots;
    std::vector<std::pair<int32_t, int64_t>> stack;
    for (int32_t s : seeds) {
        if (parent[size_t(s)] != kUnseen || ptr[size_t(s) + 1] == ptr[size_t(s)]) continue;
        parent[size_t(s)] = kRoot;
        roots.push_back(s);
        stack.assign(1, {s, ptr[size_t(s)]});
        while (!stack.empty()) {
            auto& top = stack.back();
            const int32_t u = top.first;
            if (top.second < ptr[size_t(u) + 1]) {
                const int32_t v = nbr[size_t(top.second++)];
                if (parent[size_t(v)] == kUnseen) {
                    parent[size_t(v)] = u;
                    if (child_last[size_t(u)] < 0) child_first[size_t(u)] = v;
                    else child_next[size_t(child_last[size_t(u)])] = v;
                    child_last[size_t(u)] = v;
                    stack.push_back({v, ptr[size_t(v)]});
                }
            } else {
                stack.pop_back();
            }
        }
    }
    // subtree sizes: children finish before parents in a postorder; a preorder reversed
    // (each vertex listed after its parent) gives one
    std::vector<int32_t> pre;
    pre.reserve(size_t(n));
    std::vector<int32_t> st;
    for (int32_t r : roots) {
        st.assign(1, r);
        while (!st.empty()) {
            const int32_t u = st.back();
            st.pop_back();
            pre.push_back(u);
            for (int32_t c = child_first[size_t(u)]; c >= 0; c = child_next[size_t(c)]) st.push_back(c);
        }
    }
    std::vector<int64_t> size(size_t(n), 1);
    for (auto it = pre.rbegin(); it != pre.rend(); ++it)
        if (parent[size_t(*it)] >= 0) size[size_t(parent[size_t(*it)])] += size[size_t(*it)];
    // the preorder with children in increasing subtree size (stable)
    int64_t k = 0;
    std::vector<int32_t> ch;
    for (int32_t r : roots) {
        st.assign(1, r);
        while (!st.empty()) {
            const int32_t u = st.back();
            st.pop_back();
            order[k++] = u;
            ch.clear();
            for (int32_t c = child_first[size_t(u)]; c >= 0; c = child_next[size_t(c)]) ch.push_back(c);
            std::stable_sort(ch.begin(), ch.end(),
                             [&](int32_t x, int32_t y) { return size[size_t(x)] < size[size_t(y)]; });
            for (auto it = ch.rbegin(); it != ch.rend(); ++it) st.push_back(*it);
        }
    }
    for (int32_t u = 0; u < n; ++u)
        if (ptr[size_t(u) + 1] == ptr[size_t(u)]) order[k++] = u;
    CL_REQUIRE(k == n, CL_ERR_VALUE, "internal error: order covers %lld of %d rows", (long long)k, n);
    return CL_OK;
}
