// sched_check.cpp - host-only checks of the block orders the bf16 and three-plane kernels use
// to turn a workgroup id into (head, block), and of the host rule that picks head groups.
//
// For every order (plain, descending, serpentine, grouped) and a range of grid shapes:
//   * the map is a bijection from [0, BH*nb) onto the (head, block) pairs: no block is
//     skipped or computed twice;
//   * when BH % 8 == 0, workgroup i (which the dispatcher sends to XCD i % 8) gets a head of
//     that XCD, [x*BH/8, (x+1)*BH/8), so a head's tiles stay in one L2;
//   * in the plain and grouped orders, an XCD's workgroups take the blocks heaviest first
//     (non-increasing causal work) within a head, and a group's blocks all come before the
//     next group's.
// And head_group at the bench shapes, with the resident capacities the occupancy query
// reports for those kernels on MI355X.  Prints "sched_check: all passed" on success.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "bf16_tile.hpp"
#include "sched.hpp"

using tcamd::head_group;
using tcamd::bf16t::map_block;
using tcamd::bf16t::map_block_grouped;

static int failures = 0;

#define CHECK(cond, ...)                                     \
    do {                                                     \
        if (!(cond)) {                                       \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                        \
            std::printf("\n");                               \
            if (++failures > 20) std::exit(1);               \
        }                                                    \
    } while (0)

// order: 0 plain, 1 serpentine, 2 grouped (G)
static void check_order(int BH, int nb, bool descending, int order, int G) {
    std::vector<int> seen(static_cast<size_t>(BH) * nb, 0);
    const int hpx = BH / 8;
    // per head: the last block seen (heaviest first); per XCD: the last group seen
    std::vector<int> last(BH, -1);
    std::vector<int> last_group(8, -1);
    for (int id = 0; id < BH * nb; ++id) {
        int bh = -1, b = -1;
        if (order == 2)
            map_block_grouped(id, BH, nb, G, descending, bh, b);
        else
            map_block(id, BH, nb, descending, order == 1, bh, b);
        CHECK(bh >= 0 && bh < BH && b >= 0 && b < nb,
              "BH %d nb %d order %d G %d id %d -> (%d, %d)", BH, nb, order, G, id, bh, b);
        if (bh < 0 || bh >= BH || b < 0 || b >= nb) continue;
        ++seen[static_cast<size_t>(bh) * nb + b];
        if (BH % 8 == 0) {
            CHECK(bh / hpx == id % 8, "BH %d nb %d order %d G %d: id %d (XCD %d) -> head %d",
                  BH, nb, order, G, id, id % 8, bh);
        }
        if (order != 1) {
            // heaviest first within a head: ascending blocks (key-parallel, block 0 the
            // heaviest) or descending ones (query-parallel, the last block the heaviest)
            if (last[bh] >= 0)
                CHECK(descending ? b < last[bh] : b > last[bh],
                      "BH %d nb %d order %d G %d: head %d block %d after %d", BH, nb, order, G,
                      bh, b, last[bh]);
            last[bh] = b;
        }
        if (order == 2 && G > 0 && BH % 8 == 0 && hpx % G == 0) {
            const int x = id % 8, g = (bh - x * hpx) / G;
            CHECK(g >= last_group[x], "BH %d nb %d G %d: XCD %d back to group %d after %d", BH,
                  nb, G, x, g, last_group[x]);
            last_group[x] = g;
        }
    }
    for (size_t i = 0; i < seen.size(); ++i)
        CHECK(seen[i] == 1, "BH %d nb %d order %d G %d: (head %zu, block %zu) mapped %d times",
              BH, nb, order, G, i / nb, i % nb, seen[i]);
}

int main() {
    const int bhs[] = {1, 3, 8, 12, 16, 24, 64, 96, 128, 256, 384};
    const int nbs[] = {1, 2, 7, 8, 16, 33, 64};
    for (int BH : bhs)
        for (int nb : nbs)
            for (int desc = 0; desc < 2; ++desc) {
                check_order(BH, nb, desc != 0, 0, 0);
                check_order(BH, nb, desc != 0, 1, 0);
                for (int G : {0, 1, 2, 4, 8, 16, 32}) check_order(BH, nb, desc != 0, 2, G);
            }

    // head_group(BH, nblk, resident): the groups the bench workloads get.
    // Config 3 (B16 H16 T2048 d64): bf16 dK/dV, 16 key blocks, two workgroups per CU.
    CHECK(head_group(256, 16, 512) == 8, "config 3 dK/dV: %d", head_group(256, 16, 512));
    // Config 3 forward: 16 query blocks, four workgroups per CU.
    CHECK(head_group(256, 16, 1024) == 16, "config 3 forward: %d", head_group(256, 16, 1024));
    // B16 H16 T1024 dK/dV: 8 key blocks, so a group of 8 heads fills the slots once; 16.
    CHECK(head_group(256, 8, 512) == 16, "B16 H16 T1024 dK/dV: %d", head_group(256, 8, 512));
    // B16 H16 T512 dK/dV: no group below 32 heads fills the slots twice.
    CHECK(head_group(256, 4, 512) == 0, "B16 H16 T512 dK/dV: %d", head_group(256, 4, 512));
    // Config 2 (B8 H12): 12 heads per XCD, no power of two >= 8 divides them.
    CHECK(head_group(96, 8, 512) == 0, "config 2: %d", head_group(96, 8, 512));
    // Config 4 (B2 H16 T8192 d128): 4 heads per XCD, below the smallest group.
    CHECK(head_group(32, 64, 256) == 0, "config 4: %d", head_group(32, 64, 256));
    // Heads not a multiple of the XCD count.
    CHECK(head_group(100, 64, 512) == 0, "BH 100: %d", head_group(100, 64, 512));
    // G stays below the heads per XCD (G = hpx is the plain order).
    CHECK(head_group(64, 64, 256) == 0, "BH 64: %d", head_group(64, 64, 256));

    if (failures) {
        std::printf("sched_check: %d failures\n", failures);
        return 1;
    }
    std::printf("sched_check: all passed\n");
    return 0;
}
