// Host-side tree-solve scheduler: replaces the reference's DHS ordering
// (permute_order.cpp:145-210 node_order_branch, 641-722; 971-1170
// dynamic_interleave2 / admin_dynamic2), which packs cells into 32-lane groups
// that rely on implicit warp lockstep (simulate.cu:119-189).
//
// Here a solve unit -- a few consecutive cells -- is solved by one 64-lane
// wavefront: a unit is a forest, one tree per cell, and since a wavefront
// issues the same instructions however many of its lanes have a chunk, a
// unit of several cells costs little more per round than one cell.  Each
// tree is cut into chunks: unbranched runs of at most kChunk nodes (a node
// with exactly one child continues its chunk).  A round is a set of chunks
// none of which hangs below another, up to 64 lanes; elimination walks the
// rounds from the leaves in, each chunk after every chunk hanging off its
// tail, and back substitution walks them out, with a barrier between rounds.
// Chunk ids are breadth-first so that the chunks hanging off one tail are
// consecutive LDS slots.  Each round is stored position-major (see below) so
// its lanes access memory coalesced.
#include <algorithm>
#include <cstdint>
#include <numeric>
#include <queue>
#include <stdexcept>
#include <vector>

#include "schedule.h"

namespace hx {

void build_unit_schedule(const std::vector<int>& forest_parent, int chunk_max, int lanes, int round_max,
                         UnitSchedule& out) {
    const int n = static_cast<int>(forest_parent.size());
    out = UnitSchedule();
    if (n == 0) return;
    if (forest_parent[0] != -1) throw std::runtime_error("a solve unit must start with a cell root");
    if (chunk_max < 1 || chunk_max > kChunk || round_max < chunk_max || round_max > kRoundMax)
        throw std::runtime_error("solver schedule: chunk or round size out of range");
    std::vector<int> nchild(n, 0), roots;
    for (int i = 0; i < n; ++i) {
        const int p = forest_parent[i];
        if (p < 0) {
            roots.push_back(i);
            continue;
        }
        if (p >= i) throw std::runtime_error("cell nodes must satisfy parent < child");
        nchild[p]++;
    }
    std::vector<int> cbeg(n + 1, 0);
    for (int i = 0; i < n; ++i) cbeg[i + 1] = cbeg[i] + nchild[i];
    std::vector<int> cfill(cbeg.begin(), cbeg.end() - 1), clist(std::max(n - 1, 0));
    for (int i = 0; i < n; ++i)
        if (forest_parent[i] >= 0) clist[cfill[forest_parent[i]]++] = i;

    // breadth-first chunk construction from every root: children of one chunk
    // get consecutive ids, so the child terms of a tail are summed in the same
    // order whatever else shares the unit
    struct Chunk { int head; int len; int parent; int child_begin; int child_count; std::vector<int> nodes; };
    std::vector<Chunk> chunks;
    chunks.reserve(n / 2 + roots.size());
    for (int r : roots) chunks.push_back({r, 0, -1, 0, 0, {}});
    for (size_t q = 0; q < chunks.size(); ++q) {
        int cur = chunks[q].head;
        std::vector<int> nodes{cur};
        while (nchild[cur] == 1 && static_cast<int>(nodes.size()) < chunk_max) {
            cur = clist[cbeg[cur]];
            nodes.push_back(cur);
        }
        chunks[q].nodes = nodes;
        chunks[q].len = static_cast<int>(nodes.size());
        chunks[q].child_begin = static_cast<int>(chunks.size());
        chunks[q].child_count = nchild[cur];
        for (int e = cbeg[cur]; e < cbeg[cur + 1]; ++e)
            chunks.push_back({clist[e], 0, static_cast<int>(q), 0, 0, {}});
    }
    const int nchunk = static_cast<int>(chunks.size());
    // Rounds by list scheduling, in elimination order: a chunk is ready once every
    // chunk hanging off its tail is in an earlier round, and each round takes ready
    // chunks deepest first (most chunk ancestors: the longest chain still ahead of it
    // toward its root), up to `lanes` chunks and `round_max` nodes.  A chunk that would
    // pass the node bound waits for the next round while shallower ones may still fill
    // this one.  (Grouping chunks by height instead leaves the narrow rounds near the
    // roots half empty: config 3, two cells, 47 -> 33 rounds.)  Which round a chunk
    // lands in changes no arithmetic: its inputs, its children's terms (read from
    // their slots in breadth-first order) and its results are the same.
    std::vector<int> depth(nchunk, 0);
    for (int q = 0; q < nchunk; ++q) depth[q] = chunks[q].parent < 0 ? 0 : depth[chunks[q].parent] + 1;
    std::vector<int> waiting(nchunk);
    for (int q = 0; q < nchunk; ++q) waiting[q] = chunks[q].child_count;
    auto later = [&](int x, int y) { return depth[x] != depth[y] ? depth[x] < depth[y] : x > y; };
    std::priority_queue<int, std::vector<int>, decltype(later)> ready(later);
    for (int q = 0; q < nchunk; ++q)
        if (waiting[q] == 0) ready.push(q);
    std::vector<std::vector<int>> rounds;
    int placed = 0;
    while (placed < nchunk) {
        std::vector<int> cur, held;
        int nodes = 0;
        while (!ready.empty() && static_cast<int>(cur.size()) < lanes && nodes < round_max) {
            const int q = ready.top();
            ready.pop();
            if (nodes + chunks[q].len > round_max) {
                held.push_back(q);
                continue;
            }
            cur.push_back(q);
            nodes += chunks[q].len;
        }
        for (int q : held) ready.push(q);
        if (cur.empty()) throw std::runtime_error("solver schedule: no chunk fits a round");
        for (int q : cur) {
            const int p = chunks[q].parent;
            if (p >= 0 && --waiting[p] == 0) ready.push(p);
        }
        placed += static_cast<int>(cur.size());
        // position-major storage below wants a round's chunks longest first
        std::stable_sort(cur.begin(), cur.end(), [&](int x, int y) { return chunks[x].len > chunks[y].len; });
        rounds.push_back(cur);
    }
    // back-substitution order (roots first), the order the rounds are stored in
    std::reverse(rounds.begin(), rounds.end());
    // solver order of the unit's nodes.  Inside a round the chunks are sorted by
    // length (longest first) and stored position-major: node k of every chunk
    // that has one, then node k+1, ...  Node k of lane l sits at
    // round_base + sum_{j<k} W_j + l, where W_j = number of chunks longer than j,
    // so the lanes of a round read and write contiguous memory.
    std::vector<int> round_base(rounds.size(), 0);
    out.order.reserve(n);
    for (size_t ri = 0; ri < rounds.size(); ++ri) {
        auto& r = rounds[ri];
        round_base[ri] = static_cast<int>(out.order.size());
        int maxlen = 0;
        for (int q : r) maxlen = std::max(maxlen, chunks[q].len);
        for (int k = 0; k < maxlen; ++k)
            for (int q : r)
                if (chunks[q].len > k) out.order.push_back(chunks[q].nodes[k]);
    }
    if (n > kMaxCellNodes || nchunk > kMaxCellNodes)
        throw std::runtime_error("solve unit too large for the solver schedule (max 65535 nodes and chunks)");
    for (size_t ri = 0; ri < rounds.size(); ++ri) {
        RoundInfo info{};
        info.desc_begin = static_cast<uint16_t>(out.desc.size());
        info.desc_count = static_cast<uint16_t>(rounds[ri].size());
        info.node_base = static_cast<uint16_t>(round_base[ri]);
        int cnt = 0, maxlen = 0;
        for (int q : rounds[ri]) {
            maxlen = std::max(maxlen, chunks[q].len);
            ChunkDesc d{};
            d.len = static_cast<uint8_t>(chunks[q].len);
            d.slot = static_cast<uint16_t>(q);
            d.parent_slot = chunks[q].parent >= 0 ? static_cast<uint16_t>(chunks[q].parent) : kNone;
            d.child_begin = static_cast<uint16_t>(chunks[q].child_begin);
            if (chunks[q].child_count > 255) throw std::runtime_error("node with more than 255 children");
            d.child_count = static_cast<uint8_t>(chunks[q].child_count);
            out.desc.push_back(d);
            cnt += chunks[q].len;
        }
        info.node_count = static_cast<uint16_t>(cnt);
        info.maxlen = static_cast<uint8_t>(maxlen);
        // off[k] = number of the round's nodes at positions < k (chunks sorted by length)
        int off = 0;
        for (int k = 0; k < kChunk; ++k) {
            info.off[k] = static_cast<uint16_t>(off);
            for (int q : rounds[ri]) off += chunks[q].len > k;
        }
        out.rounds.push_back(info);
    }
    // the solve kernel runs two rounds per loop trip: an odd count gets a padding
    // round with no chunks (its loads read node 0 and it writes nothing)
    if (out.rounds.size() % 2) {
        RoundInfo pad{};
        pad.node_count = 1;
        out.rounds.push_back(pad);
    }
    out.nchunk = nchunk;
    out.nround = static_cast<int>(out.rounds.size());
}

}  // namespace hx
