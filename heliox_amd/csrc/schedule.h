// Tree-solve schedule of one cell (see schedule.cpp).
#pragma once
#include <vector>

#include "hx_internal.h"

namespace hx {

struct CellSchedule {
    std::vector<int> order;          // solver position -> local node
    std::vector<ChunkDesc> desc;     // back-substitution round order
    std::vector<RoundInfo> rounds;   // [nround]
    int nchunk = 0;
    int nround = 0;
};

// local_parent: parent of each local node (-1 for local node 0, parent < child).
void build_cell_schedule(const std::vector<int>& local_parent, int chunk_max, int lanes, int round_max,
                         CellSchedule& out);

}  // namespace hx
