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

// ------------------------------------------------------------------------------------------
// LDS placement of one layer's gates for the fused packed network.  A read instruction of
// the kernel serves one half-wave (32 lanes = 32 consecutive positions) at a time, and the
// 32 lanes conflict when they read words of the same bank (word mod 32).  Gate o reads rows
// in banks ka[o] and kb[o]; a block of 32 positions is conflict-free when its gates' a banks
// are 32 distinct banks, and so are their b banks: a perfect matching of the bipartite
// multigraph (a banks x b banks, one edge per gate).  The layout is an edge colouring of that
// graph with one colour per block, every colour holding exactly 32 gates:
//   1. a bank of degree d > F (F = the region's full blocks) is split into copies of degree at
//      most F, so a proper F-colouring exists (Koenig); each gate is coloured along an
//      alternating path (the textbook bipartite edge-colouring step);
//   2. colours are balanced to exactly 32 gates by swapping along alternating paths that
//      hold one more edge of the larger colour (de Werra's equitable colouring).
// Only copies of one split bank meeting in a block conflict: at most the banks' excess over F.
// With a class size gs (> 0) every gate stays in its class's range of positions (the last
// layer, whose rows GroupSum reads by class); the positions of a class outside whole blocks
// take the gates that meet the most crowded banks, first.
namespace {

// Proper edge colouring of a bipartite multigraph with F colours (max degree <= F): per
// vertex and colour the edge of that colour (or -1); colour sizes kept for balancing.
struct Coloring {
    int F = 0;
    std::vector<int32_t> eu, ev;       // edge endpoints (left, right vertex ids)
    std::vector<int32_t> col;          // colour of each edge
    std::vector<int32_t> at_l, at_r;   // [vertex * F + colour] -> edge id or -1
    std::vector<int64_t> size;         // edges per colour

    int32_t& L(int v, int c) { return at_l[size_t(v) * size_t(F) + size_t(c)]; }
    int32_t& R(int v, int c) { return at_r[size_t(v) * size_t(F) + size_t(c)]; }
    int32_t& at(bool left, int v, int c) { return left ? L(v, c) : R(v, c); }

    // The maximal path alternating colours c1, c2, ... from vertex v (left or right side)
    // starting with its c1 edge; every vertex has at most one edge of each colour, so it is a
    // simple path when v has no c2 edge.
    std::vector<int32_t> path(bool left, int v, int c1, int c2) {
        std::vector<int32_t> p;
        int x = v, c = c1;
        while (true) {
            const int32_t e = at(left, x, c);
            if (e < 0) break;
            p.push_back(e);
            x = left ? ev[size_t(e)] : eu[size_t(e)];
            left = !left;
            c = c == c1 ? c2 : c1;
        }
        return p;
    }

    void swap_colours(const std::vector<int32_t>& p, int c1, int c2) {
        for (int32_t e : p) {
            L(eu[size_t(e)], col[size_t(e)]) = -1;
            R(ev[size_t(e)], col[size_t(e)]) = -1;
            --size[size_t(col[size_t(e)])];
        }
        for (int32_t e : p) {
            col[size_t(e)] = col[size_t(e)] == c1 ? c2 : c1;
            L(eu[size_t(e)], col[size_t(e)]) = e;
            R(ev[size_t(e)], col[size_t(e)]) = e;
            ++size[size_t(col[size_t(e)])];
        }
    }

    // Koenig's step per edge (u, v): a colour a free at u (the least used such), b free at
    // v; when a is taken at v, swapping a and b along v's a/b path frees it there (the path
    // cannot reach u, which has no a edge).
    void color_all() {
        for (size_t e = 0; e < eu.size(); ++e) {
            const int u = eu[e], v = ev[e];
            int a = -1, b = -1;
            for (int k = 0; k < F; ++k) {
                if (L(u, k) < 0 && (a < 0 || size[size_t(k)] < size[size_t(a)])) a = k;
                if (R(v, k) < 0 && b < 0) b = k;
            }
            if (R(v, a) >= 0) swap_colours(path(false, v, a, b), a, b);
            col[e] = a;
            L(u, a) = int32_t(e);
            R(v, a) = int32_t(e);
            ++size[size_t(a)];
        }
    }

    // Moves one edge from colour big to colour small along a path alternating big / small
    // that starts and ends with a big edge (one exists while big has more edges than small).
    bool move_one(int big, int small, int nl, int nr) {
        for (int side = 0; side < 2; ++side) {
            const bool left = side == 0;
            for (int v = 0; v < (left ? nl : nr); ++v) {
                if (at(left, v, big) < 0 || at(left, v, small) >= 0) continue;
                const std::vector<int32_t> p = path(left, v, big, small);
                if (p.size() % 2 == 1) {
                    swap_colours(p, big, small);
                    return true;
                }
            }
        }
        return false;
    }
};

// Positions inside a block are free for this layer's reads (only the block matters), but
// they fix the banks of the rows the next layer reads.  The block's gates, heaviest fan-out
// first, take the slot whose bank has gathered the least next-layer fan-out so far (fa: reads
// as operand a, fb: as operand b), which keeps the next layer's bank degrees level.
struct SlotBalance {
    const int32_t* fa;
    const int32_t* fb;
    int64_t la[32] = {}, lb[32] = {};

    void place(std::vector<int32_t>& blk, int64_t base, int32_t* pos) {
        constexpr int kBlock = 32;
        if (!fa) {
            for (size_t i = 0; i < blk.size(); ++i) pos[blk[i]] = int32_t(base + int64_t(i));
            return;
        }
        std::stable_sort(blk.begin(), blk.end(), [&](int32_t x, int32_t y) {
            return fa[x] + fb[x] > fa[y] + fb[y];
        });
        bool used[kBlock] = {};
        for (int32_t g : blk) {
            int best = -1;
            int64_t cost = 0;
            for (int j = 0; j < int(blk.size()); ++j) {
                if (used[j]) continue;
                const int64_t a = la[j] + fa[g], b = lb[j] + fb[g];
                const int64_t c = a * a + b * b;
                if (best < 0 || c < cost) {
                    best = j;
                    cost = c;
                }
            }
            used[best] = true;
            la[best] += fa[g];
            lb[best] += fb[g];
            pos[g] = int32_t(base + best);
        }
    }
};

// Gates idx (global ids) placed on positions [pos0, pos0 + 32 * F) as F full blocks.
bool layout_blocks(const std::vector<int32_t>& idx, const int32_t* ka, const int32_t* kb,
                   int F, int64_t pos0, int32_t* pos, SlotBalance& sb) {
    constexpr int kBanks = 32, kBlock = 32;
    // split banks: copy j of bank k takes the bank's edges j*F .. (j+1)*F - 1
    std::vector<int> cnt_a(kBanks, 0), cnt_b(kBanks, 0);
    std::vector<std::vector<int>> copy_l(kBanks), copy_r(kBanks);
    Coloring c;
    c.F = F;
    c.eu.resize(idx.size());
    c.ev.resize(idx.size());
    int nl = 0, nr = 0;
    for (size_t i = 0; i < idx.size(); ++i) {
        const int a = ka[idx[i]], b = kb[idx[i]];
        const size_t ja = size_t(cnt_a[size_t(a)]++ / F), jb = size_t(cnt_b[size_t(b)]++ / F);
        if (ja >= copy_l[size_t(a)].size()) copy_l[size_t(a)].push_back(nl++);
        if (jb >= copy_r[size_t(b)].size()) copy_r[size_t(b)].push_back(nr++);
        c.eu[i] = copy_l[size_t(a)][ja];
        c.ev[i] = copy_r[size_t(b)][jb];
    }
    c.col.assign(idx.size(), -1);
    c.at_l.assign(size_t(nl) * size_t(F), -1);
    c.at_r.assign(size_t(nr) * size_t(F), -1);
    c.size.assign(size_t(F), 0);
    c.color_all();
    while (true) {
        int big = -1, small = -1;
        for (int k = 0; k < F; ++k) {
            if (c.size[size_t(k)] > kBlock && (big < 0 || c.size[size_t(k)] > c.size[size_t(big)])) big = k;
            if (c.size[size_t(k)] < kBlock && (small < 0 || c.size[size_t(k)] < c.size[size_t(small)])) small = k;
        }
        if (big < 0 && small < 0) break;
        if (big < 0 || small < 0 || !c.move_one(big, small, nl, nr)) return false;
    }
    std::vector<std::vector<int32_t>> blocks(static_cast<size_t>(F));
    for (size_t i = 0; i < idx.size(); ++i) blocks[size_t(c.col[i])].push_back(idx[i]);
    for (int k = 0; k < F; ++k) sb.place(blocks[size_t(k)], pos0 + int64_t(k) * kBlock, pos);
    return true;
}

}  // namespace

extern "C" int cl_packed_bank_layout(const int32_t* ka, const int32_t* kb, const int32_t* fa,
                                     const int32_t* fb, int64_t n, int64_t class_size,
                                     int32_t* pos) {
    cl::clear_error();
    constexpr int kBanks = 32, kBlock = 32;
    CL_ARG(n >= 0 && n < (int64_t(1) << 30) && class_size >= 0, "bad sizes");
    CL_ARG(n == 0 || (ka && kb && pos), "null pointer argument");
    for (int64_t o = 0; o < n; ++o)
        CL_ARG(ka[o] >= 0 && ka[o] < kBanks && kb[o] >= 0 && kb[o] < kBanks,
               "gate %lld has a bank outside [0, %d)", (long long)o, kBanks);
    CL_ARG(!fa == !fb, "fa and fb are given together");
    for (int64_t o = 0; fa && o < n; ++o)
        CL_ARG(fa[o] >= 0 && fb[o] >= 0, "negative fan-out at gate %lld", (long long)o);
    SlotBalance sb{fa, fb};
    const int64_t gs = class_size > 0 ? class_size : n;
    for (int64_t lo = 0; lo < n; lo += gs) {
        const int64_t hi = std::min(n, lo + gs);
        const int64_t b0 = (lo + kBlock - 1) / kBlock, b1 = hi / kBlock;  // whole blocks
        const int F = b1 > b0 ? int(b1 - b0) : 0;
        std::vector<int32_t> gates(size_t(hi - lo));
        std::iota(gates.begin(), gates.end(), int32_t(lo));
        // positions outside whole blocks: the gates meeting the most crowded banks
        std::vector<int64_t> edge;
        for (int64_t p = lo; p < hi; ++p)
            if (F == 0 || p < b0 * kBlock || p >= b1 * kBlock) edge.push_back(p);
        if (!edge.empty()) {
            std::vector<int> da(kBanks, 0), db(kBanks, 0);
            for (int32_t o : gates) {
                ++da[size_t(ka[o])];
                ++db[size_t(kb[o])];
            }
            std::vector<char> taken(gates.size(), 0);
            for (int64_t p : edge) {
                size_t best = 0;
                int score = -1;
                for (size_t i = 0; i < gates.size(); ++i) {
                    if (taken[i]) continue;
                    const int s = da[size_t(ka[gates[i]])] + db[size_t(kb[gates[i]])];
                    if (s > score) {
                        score = s;
                        best = i;
                    }
                }
                taken[best] = 1;
                --da[size_t(ka[gates[best]])];
                --db[size_t(kb[gates[best]])];
                pos[gates[best]] = int32_t(p);
            }
            std::vector<int32_t> rest;
            for (size_t i = 0; i < gates.size(); ++i)
                if (!taken[i]) rest.push_back(gates[i]);
            gates.swap(rest);
        }
        CL_REQUIRE(F == 0 || layout_blocks(gates, ka, kb, F, b0 * kBlock, pos, sb), CL_ERR_VALUE,
                   "internal error: the block colouring of %lld gates did not balance",
                   (long long)gates.size());
    }
    // Local improvement: a gate that shares a bank with another gate of its block swaps
    // positions with a gate of its own class range in another block when that lowers the
    // layer's conflicts (the colouring leaves them where a bank is read more often than
    // there are blocks, which small class ranges make common).
    const int64_t nblk = (n + kBlock - 1) / kBlock;
    std::vector<int32_t> cnt_a(size_t(nblk) * kBanks, 0), cnt_b(size_t(nblk) * kBanks, 0);
    std::vector<int32_t> at(static_cast<size_t>(n));  // gate at each position
    for (int64_t o = 0; o < n; ++o) {
        at[size_t(pos[o])] = int32_t(o);
        ++cnt_a[size_t(pos[o] / kBlock) * kBanks + size_t(ka[o])];
        ++cnt_b[size_t(pos[o] / kBlock) * kBanks + size_t(kb[o])];
    }
    // extra reads of a (block, bank) cell holding c entries: c - 1
    auto cost_move = [&](std::vector<int32_t>& cnt, int64_t from, int64_t to, int bank_out,
                         int bank_in) {
        // change of sum max(c - 1, 0) when bank_out leaves `from` for `to` and bank_in
        // leaves `to` for `from`
        if (bank_out == bank_in) return 0;
        int d = 0;
        const size_t fo = size_t(from) * kBanks + size_t(bank_out);
        const size_t fi = size_t(from) * kBanks + size_t(bank_in);
        const size_t to_ = size_t(to) * kBanks + size_t(bank_out);
        const size_t ti = size_t(to) * kBanks + size_t(bank_in);
        d -= cnt[fo] > 1 ? 1 : 0;  // bank_out leaves from
        d += cnt[fi] >= 1 ? 1 : 0;  // bank_in joins from
        d += cnt[to_] >= 1 ? 1 : 0;  // bank_out joins to
        d -= cnt[ti] > 1 ? 1 : 0;  // bank_in leaves to
        return d;
    };
    for (int pass = 0; pass < 4; ++pass) {
        bool improved = false;
        for (int64_t g = 0; g < n; ++g) {
            const int64_t b1 = pos[g] / kBlock;
            if (cnt_a[size_t(b1) * kBanks + size_t(ka[g])] <= 1 &&
                cnt_b[size_t(b1) * kBanks + size_t(kb[g])] <= 1)
                continue;
            const int64_t lo = (g / gs) * gs, hi = std::min(n, lo + gs);
            for (int64_t p = lo; p < hi; ++p) {
                const int64_t b2 = p / kBlock;
                if (b2 == b1) continue;
                const int32_t h = at[size_t(p)];
                const int d = cost_move(cnt_a, b1, b2, ka[g], ka[h]) +
                              cost_move(cnt_b, b1, b2, kb[g], kb[h]);
                if (d >= 0) continue;
                --cnt_a[size_t(b1) * kBanks + size_t(ka[g])];
                --cnt_b[size_t(b1) * kBanks + size_t(kb[g])];
                --cnt_a[size_t(b2) * kBanks + size_t(ka[h])];
                --cnt_b[size_t(b2) * kBanks + size_t(kb[h])];
                ++cnt_a[size_t(b2) * kBanks + size_t(ka[g])];
                ++cnt_b[size_t(b2) * kBanks + size_t(kb[g])];
                ++cnt_a[size_t(b1) * kBanks + size_t(ka[h])];
                ++cnt_b[size_t(b1) * kBanks + size_t(kb[h])];
                std::swap(pos[g], pos[h]);
                at[size_t(pos[g])] = int32_t(g);
                at[size_t(pos[h])] = h;
                improved = true;
                break;
            }
        }
        if (!improved) break;
    }
    return CL_OK;
}
