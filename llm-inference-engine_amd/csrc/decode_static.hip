// Single-sequence paged decode on a device-resident, statically sized scratch
// buffer: the allocation-free twin of the single-sequence entry point.
//
// The one-row plan (row descriptor, work items, merge list) and the split
// partials live in `scratch`, a file-scope device array of
// kStaticScratchBytes. A small kernel writes the plan there from scalar
// arguments, so a call performs no allocation, no host-to-device copy and no
// host staging; then the same decode and merge kernels as the allocating
// entry point run on it, with the same partition of the row into key splits.
//
// Each device holds its own copy of the array at its own address. Host code
// never uses the array's name as a device address: the address is fetched
// once per device with hipGetSymbolAddress (InitStaticScratch, called from
// context creation with that device current) and kept per device.
//
// Calls on one device share its array, whichever context or stream makes
// them, so eager calls are ordered through a per-device event: each call's
// stream waits for the event (the previous call's end), launches, and records
// the event again, all under one lock. A call on a stream that is being
// captured into a graph skips the event (a capture may not wait on work
// recorded outside it): replays of such a graph are ordered by the stream
// they are launched on, and must not overlap eager calls on the device.
#include <hip/hip_runtime.h>

#include <mutex>

#include "kernels.h"

namespace ehip {
namespace {

constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
hipEvent_t g_scratch_done[kMaxDevices] = {};  // end of the device's last eager call

__global__ __launch_bounds__(64) void WriteRowPlan(RowDesc* rows, WorkItem* items,
                                                  int32_t* merge_rows, int32_t length,
                                                  int32_t split_len, int32_t nsplit,
                                                  int32_t kv_heads) {
  const int i = blockIdx.x * 64 + threadIdx.x;
  if (i == 0) {
    rows[0] = RowDesc{0, length, 0, nsplit};
    merge_rows[0] = 0;
  }
  const int n_items = nsplit * kv_heads;
  if (i >= n_items) return;
  // Items in key order, kv head fastest: the order the host planner gives a
  // single row (its longest-first sort keeps the shorter last range last).
  const int s = i / kv_heads;
  const int hk = i - s * kv_heads;
  const int tb = s * split_len;
  const int te = min(length, tb + split_len);
  items[i] = WorkItem{0, -1, tb, te, hk | (s << kHkBits), 0, -1, -1, -1, -1};
}

size_t Align256(size_t x) { return (x + 255) & ~size_t{255}; }

}  // namespace

hipError_t InitStaticScratch(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device]) return hipSuccess;
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  hipEvent_t done = nullptr;
  e = hipEventCreateWithFlags(&done, hipEventDisableTiming);
  if (e != hipSuccess) return e;
  g_scratch_done[device] = done;
  g_scratch_ptr[device] = ptr;
  return hipSuccess;
}

size_t StaticScratchNeed(int64_t nsplit, int kv_heads, int group, int d) {
  const size_t items = static_cast<size_t>(nsplit) * kv_heads;
  const size_t partials = items * group * (static_cast<size_t>(d) + 2) * sizeof(float);
  return 256 + Align256(items * sizeof(WorkItem)) + 256 + partials;
}

hipError_t LaunchSingleRowStatic(const DecodeParams& base, int device, int32_t length,
                                 int32_t split_len, int32_t nsplit, const Tuning& tune,
                                 QueueState* queue, hipStream_t stream) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  const int n_items = nsplit * base.kv_heads;
  if (StaticScratchNeed(nsplit, base.kv_heads, base.group, base.d) > kStaticScratchBytes)
    return hipErrorInvalidValue;
  // Held until the call's kernels are enqueued and the device event records
  // their end: calls from other threads and contexts queue behind it.
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  unsigned char* s = static_cast<unsigned char*>(g_scratch_ptr[device]);
  hipEvent_t done = g_scratch_done[device];
  if (!s || !done) return hipErrorNotInitialized;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipError_t e = hipStreamIsCapturing(stream, &cap); e != hipSuccess) return e;
  const bool ordered = cap == hipStreamCaptureStatusNone;
  if (ordered) {
    if (hipError_t e = hipStreamWaitEvent(stream, done, 0); e != hipSuccess) return e;
  }
  auto* rows = reinterpret_cast<RowDesc*>(s);
  auto* items = reinterpret_cast<WorkItem*>(s + 256);
  auto* merge = reinterpret_cast<int32_t*>(s + 256 + Align256(n_items * sizeof(WorkItem)));
  auto* part = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(merge) + 256);
  hipLaunchKernelGGL(WriteRowPlan, dim3((n_items + 63) / 64), dim3(64), 0, stream, rows, items,
                     merge, length, split_len, nsplit, base.kv_heads);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  DecodeParams p = base;
  p.rows = rows;
  p.items = items;
  p.merge_rows = merge;
  p.n_merge = nsplit > 1 ? 1 : 0;
  p.part_o = part;
  p.part_ml = part + static_cast<size_t>(n_items) * base.group * base.d;
  p.n_items = n_items;
  p.n_rows = 1;
  p.n_joint = 0;
  p.max_length = length;
  p.has_prefill = 0;
  p.head_stride = int64_t{base.bs} * base.d;
  if (hipError_t e = LaunchDecode(p, EHIP_KV_F32, tune, queue, stream); e != hipSuccess) return e;
  if (ordered) return hipEventRecord(done, stream);
  return hipSuccess;
}

}  // namespace ehip
