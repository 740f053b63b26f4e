// Run-time balancing of the per-(row block, head) attention launches over the eight XCDs.
//
// Work items sit in eight queues, one per XCD: queue x holds, head by head, a contiguous run of `per_xcd` row
// blocks, the run of head h being run (x + h) % 8, so that every queue sees every region of the sequence.
// Dispatch slot w runs on XCD w % 8 and neighbouring row blocks (which share most K / V blocks) then share that
// XCD's L2. The XCDs do not run equally fast and the items differ in work, so only the first `fixed` items of each
// queue are bound to dispatch slots (slot w takes item w / 8 of queue w % 8); the workgroups after them claim the
// remaining items through the queue counters, their own XCD's queue first and then the others in turn, so that an
// XCD that runs ahead takes over the tail of a slower one. There are twice as many claiming workgroups as
// claimable items; those that find every queue drained leave at once, and none waits for another, so every grid
// drains.
//
// The counters live in a ring of 64 slots of 8 counters in this translation unit's device memory (one copy per
// GPU, no allocation), one slot per launch, cleared by a one-wave kernel on the launch's stream just before it.
// A slot is reused only after its previous launch: every balanced launch records the slot's event on its stream
// once it is enqueued (when its Queues object is released), and the next launch that takes the slot makes its own
// stream wait for that event before clearing the counters, so launches in flight on any number of streams never
// share counters. Launches recorded inside a stream capture take their slots from a second ring of 64 (there is
// no wait and no record in a capture: a graph replays its launches in its own order), so a replay never shares
// counters with uncaptured launches; replays that overlap each other race if two of their captured launches took
// the same slot of that ring (64 captured launches apart), so replays of captured graphs must not overlap.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

namespace es {

// a claimable item for a workgroup whose home queue is `home`, or -1 once all eight queues are drained
// (wave 0 only; the result is valid in lane 0)
__device__ __forceinline__ int claim_item(int* queues, int home, int fixed, int per_queue) {
  const int l = threadIdx.x & 63;
  const int x = (home + l) & 7;
  // one round trip finds the queues that may still hold items; claims are tried on those only
  const int seen = l < 8 ? __atomic_load_n(queues + x, __ATOMIC_RELAXED) : per_queue;
  unsigned long long open = __ballot(seen < per_queue - fixed);
  int item = -1;
  if (l == 0) {
    while (open) {
      const int k = __builtin_ctzll(open);
      open &= open - 1;
      const int xq = (home + k) & 7;
      const int i = atomicAdd(queues + xq, 1);
      if (i < per_queue - fixed) {
        item = xq * per_queue + fixed + i;
        break;
      }
    }
  }
  return item;
}

// This workgroup's item as (head-major index `hd`, row block `rb`) of a grid with `per_xcd` row blocks per queue
// run and `heads` heads; false when it has none (also for padding row blocks >= n_rows). Every thread of the
// workgroup calls it (it holds a workgroup barrier when the workgroup claims).
__device__ __forceinline__ bool balanced_item(int* queues, int fixed, int per_xcd, int heads, int n_rows, int& hd,
                                              int& rb) {
  const int w = blockIdx.x, per_queue = heads * per_xcd;
  int x = w & 7, k = w >> 3;
  if (k >= fixed) {
    __shared__ int item_s;
    if (threadIdx.x < 64) {
      const int it = claim_item(queues, x, fixed, per_queue);
      if (threadIdx.x == 0) item_s = it;
    }
    __syncthreads();
    const int it = __builtin_amdgcn_readfirstlane(item_s);
    if (it < 0) return false;
    x = it / per_queue;
    k = it - x * per_queue;
  }
  hd = k / per_xcd;
  rb = ((x + hd) & 7) * per_xcd + k % per_xcd;
  return hd < heads && rb < n_rows;
}

// Head-major variant for kernels whose workgroups each stream a whole head's rows (the three-tier table
// gradients): queue x holds every row group of heads x, x + 8, ..., so that one XCD's L2 serves all workgroups of
// a head. Same claiming as above; `groups` row groups per head.
__device__ __forceinline__ bool balanced_head_item(int* queues, int fixed, int groups, int heads, int& hd, int& grp) {
  const int w = blockIdx.x, per_queue = (heads + 7) / 8 * groups;
  int x = w & 7, k = w >> 3;
  if (k >= fixed) {
    __shared__ int item_s;
    if (threadIdx.x < 64) {
      const int it = claim_item(queues, x, fixed, per_queue);
      if (threadIdx.x == 0) item_s = it;
    }
    __syncthreads();
    const int it = __builtin_amdgcn_readfirstlane(item_s);
    if (it < 0) return false;
    x = it / per_queue;
    k = it - x * per_queue;
  }
  hd = x + 8 * (k / groups);
  grp = k % groups;
  return hd < heads;
}

static __device__ int es_tile_queues[128 * 8];

static __global__ __launch_bounds__(64) void zero_queues_kernel(int* q) {
  if (threadIdx.x < 8) q[threadIdx.x] = 0;
}

// The counter ring of one GPU: the slots' device memory, one event per slot marking the end of its last launch,
// and one host lock per slot held from the slot's hand-out until that event is recorded.
struct QueueRing {
  int* base = nullptr;  // 64 slots for uncaptured launches, then 64 for captured ones
  hipEvent_t done[64] = {};
  std::mutex held[64];
  std::atomic<unsigned> seq{0};
  std::atomic<unsigned> seq_captured{0};
};

static QueueRing* queue_ring() {
  static std::atomic<QueueRing*> rings[64];
  static std::mutex init;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  QueueRing* r = rings[dev].load();
  if (r) return r;
  std::lock_guard<std::mutex> g(init);
  if ((r = rings[dev].load())) return r;
  r = new QueueRing;
  bool ok = hipGetSymbolAddress((void**)&r->base, HIP_SYMBOL(es_tile_queues)) == hipSuccess;
  for (int i = 0; ok && i < 64; ++i) ok = hipEventCreateWithFlags(&r->done[i], hipEventDisableTiming) == hipSuccess;
  if (!ok) return nullptr;  // (leaks the partial ring; the device is unusable for balanced launches anyway)
  rings[dev].store(r);
  return r;
}

// One balanced launch's counter slot. Declare it before the launch and keep it alive until the kernel is enqueued:
// releasing it (destructor, or the next balanced_launch_queues on the same object) records the slot's event on the
// launch's stream.
struct Queues {
  int* counters = nullptr;
  int fixed = 0;
  long long grid = 0;
  QueueRing* ring = nullptr;
  int slot = -1;
  bool captured = false;
  hipStream_t stream = nullptr;

  Queues() = default;
  Queues(const Queues&) = delete;
  Queues& operator=(const Queues&) = delete;
  ~Queues() { release(); }
  void release() {
    if (slot < 0) return;
    if (!captured) {
      (void)hipEventRecord(ring->done[slot], stream);
      ring->held[slot].unlock();
    }
    slot = -1;
  }
};

// Sets up one balanced launch of eight queues of per_queue items each: takes a counter slot, orders the stream
// after the slot's previous launch, clears the slot on `stream` and gives the grid size. false if the device's
// counter ring is unavailable.
static bool balanced_launch_queues(int per_queue, hipStream_t stream, Queues& out) {
  out.release();
  QueueRing* r = queue_ring();
  if (r == nullptr) return false;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const bool captured = hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
  int slot;
  if (captured) {
    slot = 64 + (int)(r->seq_captured.fetch_add(1) % 64);
  } else {
    slot = (int)(r->seq.fetch_add(1) % 64);
    r->held[slot].lock();
    if (hipStreamWaitEvent(stream, r->done[slot], 0) != hipSuccess) {
      r->held[slot].unlock();
      return false;
    }
  }
  out.ring = r;
  out.slot = slot;
  out.captured = captured;
  out.stream = stream;
  out.counters = r->base + slot * 8;
  const int claimable = (per_queue + 7) / 8;
  out.fixed = per_queue - claimable;
  out.grid = 8LL * (out.fixed + 2LL * claimable);
  hipLaunchKernelGGL(zero_queues_kernel, dim3(1), dim3(64), 0, stream, out.counters);
  return true;
}

// heads x n_rows items, n_rows split into eight runs of per_xcd (balanced_item)
static bool balanced_launch(int heads, int per_xcd, hipStream_t stream, Queues& out) {
  return balanced_launch_queues(heads * per_xcd, stream, out);
}

}  // namespace es
