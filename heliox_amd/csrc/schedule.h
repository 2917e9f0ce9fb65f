// Tree-solve schedule of one solve unit (see schedule.cpp).
#pragma once
#include <vector>

#include "hx_internal.h"

namespace hx {

struct UnitSchedule {
    std::vector<int> order;          // solver position -> local node
    std::vector<ChunkDesc> desc;     // back-substitution round order
    std::vector<RoundInfo> rounds;   // [nround]
    int nchunk = 0;
    int nround = 0;
};

// forest_parent: parent of each unit-local node (-1 for a root; parent < child),
// the unit's cells one after another, each rooted at its first node.
void build_unit_schedule(const std::vector<int>& forest_parent, int chunk_max, int lanes, int round_max,
                         UnitSchedule& out);

}  // namespace hx
