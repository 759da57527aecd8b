// sched.hpp - persistent-wave task queues for the causal attention kernels.
//
// A causal problem is a set of tasks of very different cost (query block qb of a head sees
// qb+1 key tiles).  Launching one workgroup per task leaves the placement of tasks on SIMDs
// to the dispatcher, which fixes it at launch when every task fits resident at once, and
// SIMDs then end up with 0.4x to 1.8x the average work.  Instead the kernels are
// persistent: as many workgroups as fit resident are launched, each of 4 waves (one per
// SIMD of its CU) that split every task's tile range into 4 equal parts, so the four SIMDs
// of a CU always carry equal work; workgroups pull tasks heaviest first from an atomic
// counter (dynamic longest-processing-time-first list scheduling across CUs).  The result
// of a task does not depend on which workgroup runs it, so the output is bitwise
// deterministic.
//
// Queues are per XCD: the dispatcher sends workgroup i to XCD i % 8, and when the number of
// (b,h) heads is a multiple of 8, XCD x serves only heads [x*BH/8, (x+1)*BH/8), so a head's
// K/V stays in one L2.  Otherwise a single queue serves all heads.
//
// Counters live in a file-scope __device__ array of kQueueSlots slots per kernel family;
// each launch takes the next slot from a host-side ticket, and the launch's last fetch
// resets its counter, so a slot is clean for its next use.  Launches that execute
// concurrently (different streams) therefore must not share a slot: up to kQueueSlots
// launches of one kernel family may be in flight at once.
//
// A launch captured into a HIP graph takes no slot: a graph would replay the one slot it
// captured, and two replays running at the same time (or an ordinary launch whose ticket
// wraps onto that slot) would share its counter.  Captured launches use the static
// schedule instead (slot = null): worker w runs tasks w, w + W, w + 2W, ... of the same
// heaviest-first order.  It keeps no state, and the output does not depend on the schedule.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace tcamd {

constexpr int kXcds = 8;
constexpr int kQueueSlots = 64;

// One launch's counters, one 128-byte line per counter.
struct alignas(128) QueueLine {
    unsigned v;
    unsigned pad[31];
};
struct QueueSlot {
    QueueLine next[kXcds];  // dynamic-task counter of each XCD's queue
};

// Task list of one launch as seen by one workgroup (a "worker").  Worker w of a queue
// starts with task w (no atomic at start-up); every further task comes from the atomic
// counter, offset by the number of workers.  A worker fetches exactly once per task it
// processes (and stops after a fetch returns an index >= n_tasks; a worker whose first
// task is already out of range fetches nothing), so a launch performs exactly n_tasks
// fetches on each queue, and the one that returns counter value n_tasks - 1 resets the
// counter for the slot's next launch: every other fetch of the launch has happened by then.
struct TaskQueue {
    unsigned* next;
    unsigned n_tasks;       // tasks of this worker's queue
    unsigned n_workers;     // workgroups that share this queue
    unsigned worker;        // this workgroup's index among them
    int heads_per_queue;    // (b,h) heads served by this queue
    int head_base;          // first head of this queue

    __device__ static TaskQueue bind(QueueSlot* slot, int BH, int nb, bool per_xcd) {
        TaskQueue q;
        const int x = per_xcd ? static_cast<int>(blockIdx.x % kXcds) : 0;
        q.next = slot != nullptr ? &slot->next[x].v : nullptr;  // null: static schedule
        q.heads_per_queue = per_xcd ? BH / kXcds : BH;
        q.head_base = x * q.heads_per_queue;
        q.n_tasks = static_cast<unsigned>(q.heads_per_queue) * static_cast<unsigned>(nb);
        q.n_workers = per_xcd ? gridDim.x / kXcds : gridDim.x;
        q.worker = per_xcd ? blockIdx.x / kXcds : blockIdx.x;
        return q;
    }
    __device__ unsigned first() const { return worker; }
    // Next task index of this worker after task `cur` (one thread of the workgroup calls
    // it).  Static schedule: cur + n_workers.
    __device__ unsigned fetch(unsigned cur) const {
        if (next == nullptr) return cur + n_workers;
        const unsigned c = atomicAdd(next, 1u);
        if (c + 1u == n_tasks) atomicExch(next, 0u);
        return n_workers + c;
    }
    // Task index -> (head, rank); rank 0 is the heaviest block.
    __device__ void decode(unsigned task, int& bh, int& rank) const {
        rank = static_cast<int>(task / static_cast<unsigned>(heads_per_queue));
        bh = head_base + static_cast<int>(task % static_cast<unsigned>(heads_per_queue));
    }
};

// Host side: the slot of the next launch of a kernel family.
inline unsigned next_queue_slot(std::atomic<unsigned>& ticket) {
    return ticket.fetch_add(1u, std::memory_order_relaxed) % kQueueSlots;
}

// Host side: whether work enqueued on `stream` is being captured into a graph (then the
// launch uses the static schedule).  If the query itself fails, the static schedule is
// taken: it is correct in every case.
inline bool stream_is_capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        return true;
    }
    return st != hipStreamCaptureStatusNone;
}

// Host side: the workgroups of `kernel` (block threads, lds_bytes of dynamic LDS) that the
// device holds at once, cached per (thread, kernel, device).
template <typename Kernel>
int resident_capacity(Kernel kernel, int block, size_t lds_bytes) {
    struct Entry {
        const void* fn;
        int dev;
        int cap;
    };
    static thread_local Entry cache[16] = {};
    static thread_local int cache_next = 0;
    int dev = 0;
    (void)hipGetDevice(&dev);
    const void* fn = reinterpret_cast<const void*>(kernel);
    int cap = 0;
    for (const Entry& e : cache)
        if (e.fn == fn && e.dev == dev) cap = e.cap;
    if (cap == 0) {
        // a failed query falls back to a safe guess and clears its error, which the launch
        // check after this call would otherwise report as the launch's
        int per_cu = 0, cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds_bytes) !=
            hipSuccess) {
            (void)hipGetLastError();
            per_cu = 1;
        }
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess) {
            (void)hipGetLastError();
            cus = 256;
        }
        cap = (per_cu < 1 ? 1 : per_cu) * cus;
        cache[cache_next] = Entry{fn, dev, cap};
        cache_next = (cache_next + 1) % 16;
    }
    return cap;
}

// Host side: persistent grid size: every resident workgroup slot of the device, a multiple
// of kXcds, and no more workgroups than tasks (rounded up).
template <typename Kernel>
int persistent_grid(Kernel kernel, int block, size_t lds_bytes, long long n_tasks) {
    long long g = resident_capacity(kernel, block, lds_bytes);
    const long long want = ((n_tasks + kXcds - 1) / kXcds) * kXcds;
    if (want < g) g = want;
    g = (g / kXcds) * kXcds;
    return static_cast<int>(g < kXcds ? kXcds : g);
}

// Host side: heads per group for map_block_grouped, for a grid of BH heads times nblk blocks
// that `resident` workgroups cover in more than one round: the smallest power of two G with
// 8 <= G < the heads per XCD, dividing them, whose G*nblk blocks fill the XCD's resident
// slots at least twice, so that the heaviest-first order inside a group still balances the
// CUs; 0 (no groups) if there is none.  Measured on the bf16 kernels: groups filling the
// slots only once, and groups of fewer than 8 heads, ran slower than no groups.
inline int head_group(int BH, int nblk, int resident) {
    if (BH % kXcds != 0) return 0;
    const int hpx = BH / kXcds;
    const long long slots = resident / kXcds;
    for (int G = 8; G < hpx; G *= 2)
        if (hpx % G == 0 && static_cast<long long>(G) * nblk >= 2 * slots) return G;
    return 0;
}

}  // namespace tcamd
