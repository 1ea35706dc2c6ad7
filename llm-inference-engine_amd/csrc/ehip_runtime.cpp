// C-ABI implementation: context, HBM memory, events, the per-step descriptor
// upload and the launch entry points (declared in include/ehip.h).
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "ehip.h"
#include "kernels.h"
#include "plan.h"

struct ehip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;      // the stream every call enqueues on
  hipStream_t own_stream = nullptr;  // the context's own (created at init)
  char last_error[512] = {};  // fixed storage: reporting an error allocates nothing
  ehip::Tuning tune;          // EHIP_* switches, read once at creation

  // Step descriptor: host staging (pinned, double-buffered so building step
  // n+1 never overwrites a buffer whose copy is still queued) and its device
  // image.
  void* h_stage[2] = {nullptr, nullptr};
  hipEvent_t stage_done[2] = {nullptr, nullptr};
  size_t h_stage_bytes[2] = {0, 0};
  int stage_cur = 0;
  void* d_desc = nullptr;
  size_t d_desc_bytes = 0;

  // Split-KV partials (max, sum, unnormalised output per split).
  float* d_part = nullptr;
  size_t d_part_bytes = 0;
  // Split-k partial sums of the packed linear layer.
  float* d_gemm = nullptr;
  size_t d_gemm_bytes = 0;
  int cus = 256;  // compute units of the device
  int32_t* d_err = nullptr;
  // Item-queue counters of the persistent decode kernel, in the error page
  // (zeroed at creation; every launch leaves them zero).
  ehip::QueueState queue{};

  // The uploaded step.
  bool have_step = false;
  int64_t head_stride = 0;  // kv-head stride inside a block (0: bs * d)
  ehip_geometry geom{};
  ehip::Plan plan;
  const ehip::RowDesc* d_rows = nullptr;
  const ehip::WorkItem* d_items = nullptr;
  const ehip::PrefillItem* d_prefill = nullptr;
  const int32_t* d_table = nullptr;
  const int64_t* d_slots = nullptr;
  const ehip::Q8Group* d_q8_groups = nullptr;  // INT8 append groups of the step
  const int32_t* d_q8_rows = nullptr;
  const int32_t* d_merge_rows = nullptr;
  const ehip::ItemRowsX* d_items_x = nullptr;  // null unless the plan groups beyond pairs
};

namespace {

using ehip::Plan;

int SetError(ehip_ctx* ctx, int code, const char* fmt, ...) {
  if (!ctx) return code;
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(ctx->last_error, sizeof(ctx->last_error), fmt, ap);
  va_end(ap);
  return code;
}

int HipFail(ehip_ctx* ctx, hipError_t e, const char* what) {
  const int code = (e == hipErrorOutOfMemory) ? EHIP_OUT_OF_MEMORY : EHIP_INTERNAL;
  return SetError(ctx, code, "%s: %s", what, hipGetErrorString(e));
}

#define EHIP_HIP(ctx, expr)                                  \
  do {                                                       \
    hipError_t e_ = (expr);                                  \
    if (e_ != hipSuccess) return HipFail((ctx), e_, #expr); \
  } while (0)

int CheckCtx(ehip_ctx* ctx) {
  if (!ctx) return EHIP_INVALID_ARGUMENT;
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return HipFail(ctx, e, "hipSetDevice");
  return EHIP_OK;
}

size_t Align256(size_t x) { return (x + 255) & ~size_t{255}; }

// Grows the split-partial workspace to what `plan` needs.
int EnsureWorkspace(ehip_ctx* ctx, const ehip_geometry& g, const Plan& plan) {
  const int64_t grp = g.heads / g.kv_heads;
  const size_t part_o = static_cast<size_t>(plan.partials) * grp * g.head_dim;
  const size_t part_ml = static_cast<size_t>(plan.partials) * grp * 2;
  const size_t need = Align256((part_o + part_ml) * sizeof(float));
  if (need > ctx->d_part_bytes) {
    const size_t bytes = std::max(need, ctx->d_part_bytes * 3 / 2);
    EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));  // queued kernels may use it
    if (ctx->d_part) EHIP_HIP(ctx, hipFree(ctx->d_part));
    ctx->d_part = nullptr;
    ctx->d_part_bytes = 0;
    EHIP_HIP(ctx, hipMalloc(&ctx->d_part, bytes));
    ctx->d_part_bytes = bytes;
  }
  return EHIP_OK;
}

// Packs rows | items | table ids | slots into one pinned staging buffer and
// uploads it with one async copy; records the device pointers of each part.
int UploadPlan(ehip_ctx* ctx, const ehip_geometry& g, Plan&& plan, const int32_t* d_user_table,
               int64_t head_stride = 0) {
  const size_t rows_b = Align256(plan.rows.size() * sizeof(ehip::RowDesc));
  const size_t items_b = Align256(plan.items.size() * sizeof(ehip::WorkItem));
  const size_t prefill_b = Align256(plan.prefill.size() * sizeof(ehip::PrefillItem));
  const size_t table_b = Align256(plan.table_ids.size() * sizeof(int32_t));
  const size_t slots_b = Align256(plan.slots.size() * sizeof(int64_t));
  const size_t merge_b = Align256(plan.merge_rows.size() * sizeof(int32_t));
  const size_t q8g_b = Align256(plan.q8_groups.size() * sizeof(ehip::Q8Group));
  const size_t q8r_b = Align256(plan.q8_rows.size() * sizeof(int32_t));
  const size_t itx_b = Align256(plan.items_x.size() * sizeof(ehip::ItemRowsX));
  const size_t total = std::max<size_t>(
      256, rows_b + items_b + prefill_b + table_b + slots_b + merge_b + q8g_b + q8r_b + itx_b);

  const int cur = ctx->stage_cur;
  ctx->stage_cur ^= 1;
  if (ctx->stage_done[cur]) EHIP_HIP(ctx, hipEventSynchronize(ctx->stage_done[cur]));
  if (total > ctx->h_stage_bytes[cur]) {
    const size_t bytes = std::max(total, ctx->h_stage_bytes[cur] * 3 / 2);
    if (ctx->h_stage[cur]) EHIP_HIP(ctx, hipHostFree(ctx->h_stage[cur]));
    ctx->h_stage[cur] = nullptr;
    ctx->h_stage_bytes[cur] = 0;
    EHIP_HIP(ctx, hipHostMalloc(&ctx->h_stage[cur], bytes, hipHostMallocDefault));
    ctx->h_stage_bytes[cur] = bytes;
  }
  if (total > ctx->d_desc_bytes) {
    // The old descriptor may still be read by queued kernels: wait first.
    const size_t bytes = std::max(total, ctx->d_desc_bytes * 3 / 2);
    EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->d_desc) EHIP_HIP(ctx, hipFree(ctx->d_desc));
    ctx->d_desc = nullptr;
    ctx->d_desc_bytes = 0;
    EHIP_HIP(ctx, hipMalloc(&ctx->d_desc, bytes));
    ctx->d_desc_bytes = bytes;
  }
  char* h = static_cast<char*>(ctx->h_stage[cur]);
  std::memcpy(h, plan.rows.data(), plan.rows.size() * sizeof(ehip::RowDesc));
  std::memcpy(h + rows_b, plan.items.data(), plan.items.size() * sizeof(ehip::WorkItem));
  std::memcpy(h + rows_b + items_b, plan.prefill.data(),
              plan.prefill.size() * sizeof(ehip::PrefillItem));
  std::memcpy(h + rows_b + items_b + prefill_b, plan.table_ids.data(),
              plan.table_ids.size() * sizeof(int32_t));
  std::memcpy(h + rows_b + items_b + prefill_b + table_b, plan.slots.data(),
              plan.slots.size() * sizeof(int64_t));
  std::memcpy(h + rows_b + items_b + prefill_b + table_b + slots_b, plan.merge_rows.data(),
              plan.merge_rows.size() * sizeof(int32_t));
  const size_t q8_at = rows_b + items_b + prefill_b + table_b + slots_b + merge_b;
  std::memcpy(h + q8_at, plan.q8_groups.data(), plan.q8_groups.size() * sizeof(ehip::Q8Group));
  std::memcpy(h + q8_at + q8g_b, plan.q8_rows.data(), plan.q8_rows.size() * sizeof(int32_t));
  std::memcpy(h + q8_at + q8g_b + q8r_b, plan.items_x.data(),
              plan.items_x.size() * sizeof(ehip::ItemRowsX));
  EHIP_HIP(ctx, hipMemcpyAsync(ctx->d_desc, h, total, hipMemcpyHostToDevice, ctx->stream));
  if (!ctx->stage_done[cur]) EHIP_HIP(ctx, hipEventCreateWithFlags(&ctx->stage_done[cur],
                                                                   hipEventDisableTiming));
  EHIP_HIP(ctx, hipEventRecord(ctx->stage_done[cur], ctx->stream));

  char* d = static_cast<char*>(ctx->d_desc);
  ctx->d_rows = reinterpret_cast<const ehip::RowDesc*>(d);
  ctx->d_items = reinterpret_cast<const ehip::WorkItem*>(d + rows_b);
  ctx->d_prefill = reinterpret_cast<const ehip::PrefillItem*>(d + rows_b + items_b);
  ctx->d_table = d_user_table
                     ? d_user_table
                     : reinterpret_cast<const int32_t*>(d + rows_b + items_b + prefill_b);
  ctx->d_slots = reinterpret_cast<const int64_t*>(d + rows_b + items_b + prefill_b + table_b);
  ctx->d_merge_rows =
      reinterpret_cast<const int32_t*>(d + rows_b + items_b + prefill_b + table_b + slots_b);
  ctx->d_q8_groups = reinterpret_cast<const ehip::Q8Group*>(d + q8_at);
  ctx->d_q8_rows = reinterpret_cast<const int32_t*>(d + q8_at + q8g_b);
  ctx->d_items_x = plan.items_x.empty()
                       ? nullptr
                       : reinterpret_cast<const ehip::ItemRowsX*>(d + q8_at + q8g_b + q8r_b);
  if (int rc = EnsureWorkspace(ctx, g, plan)) return rc;
  ctx->geom = g;
  ctx->plan = std::move(plan);
  ctx->have_step = true;
  ctx->head_stride = head_stride != 0 ? head_stride : int64_t{g.block_size} * g.head_dim;
  return EHIP_OK;
}

// The decode-side parameters of the uploaded step (everything but the
// fused-append rows).
ehip::DecodeParams StepDecodeParams(ehip_ctx* ctx, const float* q, const void* k_slab,
                                    const void* v_slab, float* out);

int LaunchAttention(ehip_ctx* ctx, const float* q, const void* k_slab, const void* v_slab,
                    float* out, const float* k_scale = nullptr, const float* v_scale = nullptr,
                    const float* new_k = nullptr, const float* new_v = nullptr) {
  const ehip_geometry& g = ctx->geom;
  const Plan& plan = ctx->plan;
  if (plan.items.size() > static_cast<size_t>(INT32_MAX) ||
      plan.prefill.size() > static_cast<size_t>(INT32_MAX))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "too many work items");
  if (!plan.prefill.empty()) {
    const bool aligned = reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(k_slab) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(v_slab) % 16 == 0 &&
                         ehip::BlockStride(g) % 8 == 0;
    if (!aligned)
      return SetError(ctx, EHIP_INVALID_ARGUMENT,
                      "prefill chunks need 16-byte aligned q and slabs (ehip_malloc gives 256)");
    ehip::PrefillParams pp{};
    pp.q = q;
    pp.k_slab = k_slab;
    pp.v_slab = v_slab;
    pp.out = out;
    pp.items = ctx->d_prefill;
    pp.table = ctx->d_table;
    pp.rows = ctx->d_rows;
    pp.part_o = ctx->d_part;
    pp.part_ml = ctx->d_part + static_cast<size_t>(plan.partials) * (g.heads / g.kv_heads) *
                                   g.head_dim;
    pp.err = ctx->d_err;
    pp.block_stride = ehip::BlockStride(g);
    pp.slab_blocks = g.slab_blocks;
    pp.n_items = static_cast<int32_t>(plan.prefill.size());
    pp.heads = g.heads;
    pp.kv_heads = g.kv_heads;
    pp.group = g.heads / g.kv_heads;
    pp.d = g.head_dim;
    pp.bs = g.block_size;
    pp.scale_log2 = g.scale * 1.4426950408889634f;
    hipError_t e = hipSuccess;
    if (!ehip::LaunchPrefillMfma(pp, ctx->stream, &e))
      return SetError(ctx, EHIP_INTERNAL, "prefill plan for a shape the kernel does not cover");
    EHIP_HIP(ctx, e);
  }
  if (plan.items.empty() && plan.merge_rows.empty()) return EHIP_OK;
  ehip::DecodeParams p = StepDecodeParams(ctx, q, k_slab, v_slab, out);
  p.k_scale = k_scale;
  p.v_scale = v_scale;
  p.new_k = new_k;
  p.new_v = new_v;
  EHIP_HIP(ctx, ehip::LaunchDecode(p, g.kv_dtype, ctx->tune, &ctx->queue, ctx->stream));
  return EHIP_OK;
}

ehip::DecodeParams StepDecodeParams(ehip_ctx* ctx, const float* q, const void* k_slab,
                                    const void* v_slab, float* out) {
  const ehip_geometry& g = ctx->geom;
  const Plan& plan = ctx->plan;
  ehip::DecodeParams p{};
  p.q = q;
  p.k_slab = k_slab;
  p.v_slab = v_slab;
  p.out = out;
  p.rows = ctx->d_rows;
  p.items = ctx->d_items;
  p.table = ctx->d_table;
  const int64_t grp = g.heads / g.kv_heads;
  p.part_o = ctx->d_part;
  p.part_ml = ctx->d_part + static_cast<size_t>(plan.partials) * grp * g.head_dim;
  p.err = ctx->d_err;
  p.block_stride = ehip::BlockStride(g);
  p.head_stride = ctx->head_stride;
  p.slab_blocks = g.slab_blocks;
  p.n_items = static_cast<int32_t>(plan.items.size());
  p.n_rows = static_cast<int32_t>(plan.rows.size());
  p.merge_rows = ctx->d_merge_rows;
  p.n_merge = static_cast<int32_t>(plan.merge_rows.size());
  p.n_joint = static_cast<int32_t>(plan.joint_items);
  p.joint_rows = plan.joint_rows;
  p.items_x = ctx->d_items_x;
  p.heads = g.heads;
  p.kv_heads = g.kv_heads;
  p.group = static_cast<int32_t>(grp);
  p.d = g.head_dim;
  p.bs = g.block_size;
  p.scale_log2 = g.scale * 1.4426950408889634f;
  p.max_length = plan.max_length;
  p.has_prefill = plan.prefill.empty() ? 0 : 1;
  p.slots = ctx->d_slots;
  return p;
}

bool NonNull(const void* a) { return a != nullptr; }

}  // namespace

extern "C" {

int ehip_device_count(int* out) {
  if (!out) return EHIP_INVALID_ARGUMENT;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
  *out = n;
  return EHIP_OK;
}

int ehip_init(int device, ehip_ctx** out) {
  if (!out) return EHIP_INVALID_ARGUMENT;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return EHIP_FAILED_PRECONDITION;
  if (device < 0 || device >= n) return EHIP_INVALID_ARGUMENT;
  ehip_ctx* ctx = new (std::nothrow) ehip_ctx;
  if (!ctx) return EHIP_OUT_OF_MEMORY;
  ctx->device = device;
  ctx->tune = ehip::ReadTuning();
  int rc = EHIP_OK;
  do {
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) { rc = HipFail(ctx, e, "hipSetDevice"); break; }
    // Default priority (a non-default priority stream has hung on this pool).
    e = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
    ctx->stream = ctx->own_stream;
    if (e != hipSuccess) { rc = HipFail(ctx, e, "hipStreamCreate"); break; }
    // Word 0 holds the range flags; from word 1024 the decode item
    // queue: kItemQueues ticket counters kQueueStride words apart, then the
    // wavefronts-done counter.
    constexpr size_t kQueueWord = 1024;
    constexpr size_t kPageBytes =
        4 * (kQueueWord + (ehip::kItemQueues + 1) * size_t{ehip::kQueueStride});
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
        cus > 0)
      ctx->cus = cus;
    e = hipMalloc(&ctx->d_err, kPageBytes);
    if (e != hipSuccess) { rc = HipFail(ctx, e, "hipMalloc(err)"); break; }
    e = hipMemset(ctx->d_err, 0, kPageBytes);
    if (e != hipSuccess) { rc = HipFail(ctx, e, "hipMemset(err)"); break; }
    uint32_t* words = reinterpret_cast<uint32_t*>(ctx->d_err);
    ctx->queue.d_counters = words + kQueueWord;
    ctx->queue.d_done = words + kQueueWord + size_t{ehip::kItemQueues} * ehip::kQueueStride;
    // The device address of the allocation-free entry point's static scratch
    // (fetched once per device, with the device current).
    e = ehip::InitStaticScratch(device);
    if (e != hipSuccess) { rc = HipFail(ctx, e, "hipGetSymbolAddress(scratch)"); break; }
  } while (false);
  if (rc != EHIP_OK) {
    ehip_destroy(ctx);
    return rc;
  }
  *out = ctx;
  return EHIP_OK;
}

int ehip_destroy(ehip_ctx* ctx) {
  if (!ctx) return EHIP_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  for (int i = 0; i < 2; ++i) {
    if (ctx->stage_done[i]) (void)hipEventDestroy(ctx->stage_done[i]);
    if (ctx->h_stage[i]) (void)hipHostFree(ctx->h_stage[i]);
  }
  if (ctx->d_desc) (void)hipFree(ctx->d_desc);
  if (ctx->d_part) (void)hipFree(ctx->d_part);
  if (ctx->d_gemm) (void)hipFree(ctx->d_gemm);
  if (ctx->d_err) (void)hipFree(ctx->d_err);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
  return EHIP_OK;
}

int ehip_last_error(const ehip_ctx* ctx, char* buf, size_t n) {
  if (!ctx || !buf || n == 0) return EHIP_INVALID_ARGUMENT;
  std::snprintf(buf, n, "%s", ctx->last_error);
  return EHIP_OK;
}

int ehip_sync(ehip_ctx* ctx) {
  if (int rc = CheckCtx(ctx)) return rc;
  EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));
  int32_t flags = 0;
  EHIP_HIP(ctx, hipMemcpy(&flags, ctx->d_err, sizeof(flags), hipMemcpyDeviceToHost));
  // Every persistent decode launch leaves its queue counters zero. Non-zero
  // counters after the stream drained mean two launches on this context
  // overlapped (or one was cut short): later launches would skip items, so
  // the counters are cleared and the step reported as failed.
  const size_t queue_bytes = sizeof(uint32_t) * (size_t{ehip::kItemQueues} + 1) * ehip::kQueueStride;
  std::vector<uint32_t> queue(queue_bytes / sizeof(uint32_t));
  EHIP_HIP(ctx, hipMemcpy(queue.data(), ctx->queue.d_counters, queue_bytes, hipMemcpyDeviceToHost));
  bool dirty = false;
  for (int k = 0; k <= ehip::kItemQueues; ++k) dirty = dirty || queue[static_cast<size_t>(k) * ehip::kQueueStride];
  if (dirty) {
    EHIP_HIP(ctx, hipMemset(ctx->queue.d_counters, 0, queue_bytes));
    return SetError(ctx, EHIP_INTERNAL,
                    "decode item-queue counters were left non-zero (overlapping launches on one "
                    "context?); cleared, and the outputs since the last sync are suspect");
  }
  if (flags != 0) {
    EHIP_HIP(ctx, hipMemset(ctx->d_err, 0, sizeof(flags)));
    return SetError(ctx, EHIP_INVALID_ARGUMENT,
                    "device range check failed (flags=%d: %s%s); the offending rows were skipped",
                    flags, (flags & ehip::kErrSlotRange) ? "slot outside slab " : "",
                    (flags & ehip::kErrBlockRange) ? "block id outside slab" : "");
  }
  return EHIP_OK;
}

int ehip_set_stream(ehip_ctx* ctx, void* stream) {
  if (int rc = CheckCtx(ctx)) return rc;
  hipStream_t next = stream ? static_cast<hipStream_t>(stream) : ctx->own_stream;
  if (next == ctx->stream) return EHIP_OK;
  // The context owns one descriptor arena, one split workspace and one set of
  // queue counters: work still queued on the old stream must finish before
  // anything runs on the new one, or two launches would share them.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  EHIP_HIP(ctx, hipStreamIsCapturing(ctx->stream, &cap));
  if (cap != hipStreamCaptureStatusNone)
    return SetError(ctx, EHIP_FAILED_PRECONDITION,
                    "the context's stream is being captured: end the capture before switching");
  EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));
  ctx->stream = next;
  return EHIP_OK;
}

int ehip_malloc(ehip_ctx* ctx, int64_t bytes, void** d_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!d_out || bytes < 0) return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad malloc arguments");
  *d_out = nullptr;
  void* p = nullptr;
  const size_t n = std::max<size_t>(256, Align256(static_cast<size_t>(bytes)));
  EHIP_HIP(ctx, hipMalloc(&p, n));  // hipMalloc returns >= 256-byte aligned memory
  hipError_t e = hipMemsetAsync(p, 0, n, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return HipFail(ctx, e, "zero-fill");
  }
  *d_out = p;
  return EHIP_OK;
}

int ehip_free(ehip_ctx* ctx, void* d_ptr) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!d_ptr) return EHIP_OK;
  EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));
  EHIP_HIP(ctx, hipFree(d_ptr));
  return EHIP_OK;
}

int ehip_copy_to_device(ehip_ctx* ctx, void* d_dst, const void* h_src, int64_t bytes) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (bytes < 0 || (bytes > 0 && (!d_dst || !h_src)))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad copy arguments");
  if (bytes == 0) return EHIP_OK;
  EHIP_HIP(ctx, hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream));
  EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return EHIP_OK;
}

int ehip_copy_to_host(ehip_ctx* ctx, void* h_dst, const void* d_src, int64_t bytes) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (bytes < 0 || (bytes > 0 && (!h_dst || !d_src)))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad copy arguments");
  if (bytes == 0) return EHIP_OK;
  EHIP_HIP(ctx, hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return EHIP_OK;
}

int ehip_copy_device(ehip_ctx* ctx, void* d_dst, const void* d_src, int64_t bytes) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (bytes < 0 || (bytes > 0 && (!d_dst || !d_src)))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad copy arguments");
  if (bytes == 0) return EHIP_OK;
  EHIP_HIP(ctx, hipMemcpyAsync(d_dst, d_src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return EHIP_OK;
}

int ehip_fill_normal(ehip_ctx* ctx, void* d_dst, int64_t n, int32_t dtype, float mean,
                     float stddev, uint64_t seed) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (n < 0 || (n > 0 && !d_dst) ||
      (dtype != EHIP_KV_F32 && dtype != EHIP_KV_BF16 && dtype != EHIP_KV_FP8))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad fill arguments");
  EHIP_HIP(ctx, ehip::LaunchFillNormal(d_dst, n, dtype, mean, stddev, seed, ctx->stream));
  return EHIP_OK;
}


int ehip_event_create(ehip_ctx* ctx, void** ev_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ev_out) return SetError(ctx, EHIP_INVALID_ARGUMENT, "null event out");
  hipEvent_t ev = nullptr;
  EHIP_HIP(ctx, hipEventCreate(&ev));
  *ev_out = ev;
  return EHIP_OK;
}

int ehip_event_destroy(ehip_ctx* ctx, void* ev) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (ev) EHIP_HIP(ctx, hipEventDestroy(static_cast<hipEvent_t>(ev)));
  return EHIP_OK;
}

int ehip_event_record(ehip_ctx* ctx, void* ev) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ev) return SetError(ctx, EHIP_INVALID_ARGUMENT, "null event");
  EHIP_HIP(ctx, hipEventRecord(static_cast<hipEvent_t>(ev), ctx->stream));
  return EHIP_OK;
}

int ehip_event_elapsed_ms(ehip_ctx* ctx, void* ev_start, void* ev_end, float* ms_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ev_start || !ev_end || !ms_out) return SetError(ctx, EHIP_INVALID_ARGUMENT, "null event");
  EHIP_HIP(ctx, hipEventSynchronize(static_cast<hipEvent_t>(ev_end)));
  EHIP_HIP(ctx, hipEventElapsedTime(ms_out, static_cast<hipEvent_t>(ev_start),
                                    static_cast<hipEvent_t>(ev_end)));
  return EHIP_OK;
}

// ----------------------------------------------------- reference kernels --

int ehip_kv_scatter_f32(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                        const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads,
                        int64_t d, int64_t block_size, int64_t slab_blocks, float* d_k_slab,
                        float* d_v_slab) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (t_dim < 0 || kv_heads < 1 || d < 1 || block_size < 1 || slab_blocks < 1 ||
      kv_heads > INT32_MAX || d > INT32_MAX || block_size > INT32_MAX)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad scatter geometry");
  if (t_dim == 0) return EHIP_OK;
  if (!d_src_k || !d_src_v || !d_slot_mapping || !d_k_slab || !d_v_slab)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null scatter operand");
  EHIP_HIP(ctx, ehip::LaunchKvScatter(d_src_k, d_src_v, d_slot_mapping, t_dim,
                                      static_cast<int32_t>(kv_heads), static_cast<int32_t>(d),
                                      static_cast<int32_t>(block_size), slab_blocks, d_k_slab,
                                      d_v_slab, EHIP_KV_F32, ctx->d_err, ctx->stream));
  return EHIP_OK;
}

int ehip_kv_scatter_bf16(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                         const int64_t* d_slot_mapping, int64_t t_dim, int64_t kv_heads,
                         int64_t d, int64_t block_size, int64_t slab_blocks,
                         uint16_t* d_k_slab, uint16_t* d_v_slab) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (t_dim < 0 || kv_heads < 1 || d < 1 || block_size < 1 || slab_blocks < 1 ||
      kv_heads > INT32_MAX || d > INT32_MAX || block_size > INT32_MAX)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad scatter geometry");
  if (t_dim == 0) return EHIP_OK;
  if (!d_src_k || !d_src_v || !d_slot_mapping || !d_k_slab || !d_v_slab)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null scatter operand");
  EHIP_HIP(ctx, ehip::LaunchKvScatter(d_src_k, d_src_v, d_slot_mapping, t_dim,
                                      static_cast<int32_t>(kv_heads), static_cast<int32_t>(d),
                                      static_cast<int32_t>(block_size), slab_blocks, d_k_slab,
                                      d_v_slab, EHIP_KV_BF16, ctx->d_err, ctx->stream));
  return EHIP_OK;
}

int ehip_kv_gather_f32(ehip_ctx* ctx, const float* d_k_slab, const float* d_v_slab,
                       const int32_t* d_block_table, int64_t block_size, int64_t length,
                       int64_t kv_heads, int64_t d, int64_t slab_blocks, float* d_out_k,
                       float* d_out_v) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (length < 0 || kv_heads < 1 || d < 1 || block_size < 1 || slab_blocks < 1 ||
      kv_heads > INT32_MAX || d > INT32_MAX || block_size > INT32_MAX)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "bad gather geometry");
  if (length == 0) return EHIP_OK;  // the reference returns early (kv_gather.cpp:66-68)
  if (!d_k_slab || !d_v_slab || !d_block_table || !d_out_k || !d_out_v)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null gather operand");
  EHIP_HIP(ctx, ehip::LaunchKvGather(d_k_slab, d_v_slab, d_block_table,
                                     static_cast<int32_t>(block_size), length,
                                     static_cast<int32_t>(kv_heads), static_cast<int32_t>(d),
                                     slab_blocks, d_out_k, d_out_v, ctx->d_err, ctx->stream));
  return EHIP_OK;
}

int ehip_paged_decode_attention_f32(ehip_ctx* ctx, const float* d_q, const float* d_k_slab,
                                    const float* d_v_slab, const int32_t* d_block_table,
                                    int64_t num_blocks, int64_t length, int64_t heads,
                                    int64_t kv_heads, int64_t d, int64_t block_size,
                                    int64_t block_stride, int64_t slab_blocks, float scale,
                                    float* d_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (heads > INT32_MAX || kv_heads > INT32_MAX || d > INT32_MAX || block_size > INT32_MAX)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "geometry out of range");
  ehip_geometry g{static_cast<int32_t>(heads), static_cast<int32_t>(kv_heads),
                  static_cast<int32_t>(d),     static_cast<int32_t>(block_size),
                  EHIP_KV_F32,                 0,
                  slab_blocks,                 block_stride,
                  scale};
  if (!NonNull(d_q) || !NonNull(d_k_slab) || !NonNull(d_v_slab) || !NonNull(d_block_table) ||
      !NonNull(d_out))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null decode operand");
  Plan plan;
  std::string err;
  if (int rc = ehip::BuildSingleRowPlan(g, length, num_blocks, ctx->tune, &plan, &err))
    return SetError(ctx, rc, "%s", err.c_str());
  if (int rc = UploadPlan(ctx, g, std::move(plan), d_block_table)) return rc;
  return LaunchAttention(ctx, d_q, d_k_slab, d_v_slab, d_out);
}

int ehip_paged_decode_attention_f32_noalloc(ehip_ctx* ctx, const float* d_q,
                                            const float* d_k_slab, const float* d_v_slab,
                                            const int32_t* d_block_table, int64_t num_blocks,
                                            int64_t length, int64_t heads, int64_t kv_heads,
                                            int64_t d, int64_t block_size, int64_t block_stride,
                                            int64_t slab_blocks, float scale, float* d_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (heads > INT32_MAX || kv_heads > INT32_MAX || d > INT32_MAX || block_size > INT32_MAX)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "geometry out of range");
  const ehip_geometry g{static_cast<int32_t>(heads), static_cast<int32_t>(kv_heads),
                        static_cast<int32_t>(d),     static_cast<int32_t>(block_size),
                        EHIP_KV_F32,                 0,
                        slab_blocks,                 block_stride,
                        scale};
  // The same checks as the allocating entry point, without building a plan
  // on the host or a message string.
  if (int rc = ehip::ValidateGeometry(g, nullptr))
    return SetError(ctx, rc, "invalid geometry (heads=%d kv_heads=%d d=%d block_size=%d)", g.heads,
                    g.kv_heads, g.head_dim, g.block_size);
  if (!NonNull(d_q) || !NonNull(d_k_slab) || !NonNull(d_v_slab) || !NonNull(d_block_table) ||
      !NonNull(d_out))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null decode operand");
  if (length < 1 || length > (int64_t{1} << 30))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "length=%lld out of range",
                    static_cast<long long>(length));
  if ((length + block_size - 1) / block_size > num_blocks)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "ceil(length/bs) exceeds num_blocks=%lld",
                    static_cast<long long>(num_blocks));
  const int32_t split_len = ehip::SingleRowSplitTokens(g, length, ctx->tune);
  const int64_t nsplit = (length + split_len - 1) / split_len;
  const int group = g.heads / g.kv_heads;
  const size_t need = ehip::StaticScratchNeed(nsplit, g.kv_heads, group, g.head_dim);
  if (need > ehip::kStaticScratchBytes)
    return SetError(ctx, EHIP_RESOURCE_EXHAUSTED,
                    "the row needs %zu bytes of scratch (%lld key splits x %d query heads); the "
                    "static scratch holds %zu: use ehip_paged_decode_attention_f32",
                    need, static_cast<long long>(nsplit), g.heads, ehip::kStaticScratchBytes);
  ehip::DecodeParams p{};
  p.q = d_q;
  p.k_slab = d_k_slab;
  p.v_slab = d_v_slab;
  p.out = d_out;
  p.table = d_block_table;
  p.err = ctx->d_err;
  p.block_stride = ehip::BlockStride(g);
  p.head_stride = int64_t{g.block_size} * g.head_dim;
  p.slab_blocks = g.slab_blocks;
  p.heads = g.heads;
  p.kv_heads = g.kv_heads;
  p.group = group;
  p.d = g.head_dim;
  p.bs = g.block_size;
  p.scale_log2 = g.scale * 1.4426950408889634f;
  EHIP_HIP(ctx, ehip::LaunchSingleRowStatic(p, ctx->device, static_cast<int32_t>(length),
                                            split_len, static_cast<int32_t>(nsplit), ctx->tune,
                                            &ctx->queue, ctx->stream));
  return EHIP_OK;
}

namespace {
// kernels::PrefillAttentionF32 / DecodeAttentionF32 over a contiguous
// [Hkv, L, d] cache: one sequence whose "blocks" are consecutive 16-row runs
// of each kv head (identity table, block stride 16 d, kv-head stride L d),
// planned and launched like any step with T rows at the end of L keys.
int ContiguousAttention(ehip_ctx* ctx, const float* d_q, const float* d_k, const float* d_v,
                        float* d_out, int64_t t_dim, int64_t heads, int64_t kv_heads, int64_t d,
                        int64_t l_dim, float scale) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (heads < 1 || kv_heads < 1 || d < 1 || heads > INT32_MAX || kv_heads > INT32_MAX ||
      d > INT32_MAX || heads % kv_heads != 0)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "heads=%lld kv_heads=%lld d=%lld invalid",
                    static_cast<long long>(heads), static_cast<long long>(kv_heads),
                    static_cast<long long>(d));
  if (t_dim < 1 || l_dim < t_dim || l_dim > (int64_t{1} << 30))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "need 1 <= T (%lld) <= L (%lld) <= 2^30",
                    static_cast<long long>(t_dim), static_cast<long long>(l_dim));
  if (!d_q || !d_k || !d_v || !d_out)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null attention operand");
  constexpr int32_t kRun = 16;
  const int64_t nblk = (l_dim + kRun - 1) / kRun;
  const ehip_geometry g{static_cast<int32_t>(heads), static_cast<int32_t>(kv_heads),
                        static_cast<int32_t>(d), kRun, EHIP_KV_F32, 0, nblk, kRun * d, scale};
  std::vector<int32_t> ids(static_cast<size_t>(nblk));
  for (int64_t i = 0; i < nblk; ++i) ids[static_cast<size_t>(i)] = static_cast<int32_t>(i);
  const int32_t qlen = static_cast<int32_t>(t_dim);
  const int32_t offsets[2] = {0, static_cast<int32_t>(nblk)};
  const ehip_step_desc s{1, 0, &qlen, &l_dim, offsets, ids.data(), nullptr};
  Plan plan;
  std::string err;
  if (int rc = ehip::BuildPlan(g, s, ctx->tune, &plan, &err, 0, /*head_major=*/true))
    return SetError(ctx, rc, "%s", err.c_str());
  if (int rc = UploadPlan(ctx, g, std::move(plan), nullptr, l_dim * d)) return rc;
  return LaunchAttention(ctx, d_q, d_k, d_v, d_out);
}
}  // namespace

int ehip_prefill_attention_f32(ehip_ctx* ctx, const float* d_q, const float* d_k,
                               const float* d_v, float* d_out, int64_t t_dim, int64_t heads,
                               int64_t kv_heads, int64_t d, int64_t l_dim, float scale) {
  return ContiguousAttention(ctx, d_q, d_k, d_v, d_out, t_dim, heads, kv_heads, d, l_dim, scale);
}

int ehip_decode_attention_f32(ehip_ctx* ctx, const float* d_q, const float* d_k, const float* d_v,
                              float* d_out, int64_t heads, int64_t kv_heads, int64_t d,
                              int64_t l_dim, float scale) {
  return ContiguousAttention(ctx, d_q, d_k, d_v, d_out, 1, heads, kv_heads, d, l_dim, scale);
}

namespace {
bool WeightDtypeOk(int32_t t) {
  return t == EHIP_WEIGHT_F32 || t == EHIP_WEIGHT_BF16 || t == EHIP_WEIGHT_F16;
}
}  // namespace

int ehip_pack_weight_panels(ehip_ctx* ctx, const void* d_w, int32_t weight_dtype, int64_t n,
                            int64_t k, void* d_wp) {
  if (int rc = CheckCtx(ctx)) return rc;
  // The reference CHECKs n, k >= 1 and non-null operands (src/kernels/gemm.cpp:123-125).
  if (n < 1 || k < 1 || n > (int64_t{1} << 31) || k > (int64_t{1} << 31))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "pack: n=%lld k=%lld must be in [1, 2^31]",
                    static_cast<long long>(n), static_cast<long long>(k));
  if (!WeightDtypeOk(weight_dtype))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "pack: weight_dtype=%d is not F32/BF16/F16",
                    weight_dtype);
  if (!d_w || !d_wp) return SetError(ctx, EHIP_INVALID_ARGUMENT, "pack: null operand");
  EHIP_HIP(ctx, ehip::LaunchPackWeightPanels(d_w, weight_dtype, n, k, d_wp, ctx->stream));
  return EHIP_OK;
}

int ehip_packed_gemm(ehip_ctx* ctx, const float* d_x, int64_t m, int64_t k, const void* d_wp,
                     int32_t weight_dtype, int64_t n, const float* d_bias, float* d_y) {
  if (int rc = CheckCtx(ctx)) return rc;
  // The reference CHECKs m, k, n >= 1 and a supported dtype (src/kernels/gemm.h:76-78).
  if (m < 1 || k < 1 || n < 1 || m > (int64_t{1} << 31) || k > (int64_t{1} << 31) ||
      n > (int64_t{1} << 31))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "gemm: m=%lld k=%lld n=%lld must be in [1, 2^31]",
                    static_cast<long long>(m), static_cast<long long>(k),
                    static_cast<long long>(n));
  if (!WeightDtypeOk(weight_dtype))
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "gemm: weight_dtype=%d is not F32/BF16/F16",
                    weight_dtype);
  if (!d_x || !d_wp || !d_y) return SetError(ctx, EHIP_INVALID_ARGUMENT, "gemm: null operand");
  if (reinterpret_cast<uintptr_t>(d_wp) % 16 != 0)
    return SetError(ctx, EHIP_INVALID_ARGUMENT,
                    "gemm: the packed weight must be 16-byte aligned (ehip_malloc gives 256)");
  ehip::GemmParams p{};
  ehip::PlanPackedGemm(m, k, n, weight_dtype, ctx->cus, &p);
  p.x = d_x;
  p.wp = d_wp;
  p.bias = d_bias;
  p.y = d_y;
  p.x_vec = (k % 4 == 0 && reinterpret_cast<uintptr_t>(d_x) % 16 == 0) ? 1 : 0;
  {
    // x's bf16 planes, then (split k) the partial sums, 256 bytes apart.
    const size_t planes = (ehip::PackedGemmPlaneBytes(p) + 255) & ~size_t{255};
    const size_t partial = p.splits > 1 ? static_cast<size_t>(p.splits) * static_cast<size_t>(m) *
                                              static_cast<size_t>(n) * sizeof(float)
                                        : 0;
    const size_t need = planes + partial;
    if (need > ctx->d_gemm_bytes) {
      const size_t bytes = std::max(need, ctx->d_gemm_bytes * 3 / 2);
      EHIP_HIP(ctx, hipStreamSynchronize(ctx->stream));  // queued calls may use it
      if (ctx->d_gemm) EHIP_HIP(ctx, hipFree(ctx->d_gemm));
      ctx->d_gemm = nullptr;
      ctx->d_gemm_bytes = 0;
      EHIP_HIP(ctx, hipMalloc(&ctx->d_gemm, bytes));
      ctx->d_gemm_bytes = bytes;
    }
    p.xp = reinterpret_cast<uint16_t*>(ctx->d_gemm);
    p.part = p.splits > 1 ? reinterpret_cast<float*>(reinterpret_cast<char*>(ctx->d_gemm) + planes)
                          : nullptr;
  }
  EHIP_HIP(ctx, ehip::LaunchPackedGemm(p, weight_dtype, ctx->stream));
  return EHIP_OK;
}

int ehip_prefill_attention_varlen_f32(ehip_ctx* ctx, const float* d_q,
                                      const int32_t* h_cu_seqlens, int64_t num_seqs,
                                      const float* const* h_k_seqs,
                                      const float* const* h_v_seqs, const int64_t* h_l_dims,
                                      float* d_out, int64_t heads, int64_t kv_heads, int64_t d,
                                      float scale) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (num_seqs < 0 || num_seqs > INT32_MAX)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "num_seqs=%lld out of range",
                    static_cast<long long>(num_seqs));
  if (num_seqs == 0) return EHIP_OK;  // the reference's B == 0 no-op
  if (!h_cu_seqlens || !h_k_seqs || !h_v_seqs || !h_l_dims || !d_q || !d_out)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null varlen operand");
  if (heads < 1 || kv_heads < 1 || d < 1 || heads > INT32_MAX || kv_heads > INT32_MAX ||
      d > INT32_MAX || heads % kv_heads != 0)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "heads=%lld kv_heads=%lld d=%lld invalid",
                    static_cast<long long>(heads), static_cast<long long>(kv_heads),
                    static_cast<long long>(d));
  if (h_cu_seqlens[0] != 0)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "cu_seqlens[0]=%d must be 0", h_cu_seqlens[0]);
  // All-or-nothing: every sequence is checked before the first launch.
  for (int64_t b = 0; b < num_seqs; ++b) {
    const int64_t T = int64_t{h_cu_seqlens[b + 1]} - h_cu_seqlens[b];
    const int64_t L = h_l_dims[b];
    if (T < 1 || L < T || L > (int64_t{1} << 30))
      return SetError(ctx, EHIP_INVALID_ARGUMENT,
                      "sequence %lld: need 1 <= T (%lld) <= L (%lld) <= 2^30",
                      static_cast<long long>(b), static_cast<long long>(T),
                      static_cast<long long>(L));
    if (!h_k_seqs[b] || !h_v_seqs[b])
      return SetError(ctx, EHIP_INVALID_ARGUMENT, "sequence %lld: null K/V",
                      static_cast<long long>(b));
  }
  const int64_t row = heads * d;
  for (int64_t b = 0; b < num_seqs; ++b) {
    const int64_t r0 = h_cu_seqlens[b];
    const int64_t T = int64_t{h_cu_seqlens[b + 1]} - r0;
    if (int rc = ContiguousAttention(ctx, d_q + r0 * row, h_k_seqs[b], h_v_seqs[b],
                                     d_out + r0 * row, T, heads, kv_heads, d, h_l_dims[b], scale))
      return rc;
  }
  return EHIP_OK;
}

namespace {
int BatchedDecode(ehip_ctx* ctx, int kv_dtype, const float* d_q, const void* d_k_slab,
                  const void* d_v_slab, const int32_t* const* h_block_tables,
                  const int64_t* h_lengths, int64_t num_seqs, int64_t heads, int64_t kv_heads,
                  int64_t d, int64_t block_size, int64_t block_stride, int64_t slab_blocks,
                  float scale, float* d_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (num_seqs < 0 || num_seqs > INT32_MAX || heads > INT32_MAX || kv_heads > INT32_MAX ||
      d > INT32_MAX || block_size > INT32_MAX)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "geometry out of range");
  ehip_geometry g{static_cast<int32_t>(heads), static_cast<int32_t>(kv_heads),
                  static_cast<int32_t>(d),     static_cast<int32_t>(block_size),
                  kv_dtype,                    0,
                  slab_blocks,                 block_stride,
                  scale};
  std::string err;
  if (int rc = ehip::ValidateGeometry(g, &err)) return SetError(ctx, rc, "%s", err.c_str());
  if (num_seqs == 0) return EHIP_OK;  // the reference's B == 0 no-op
  if (!h_block_tables || !h_lengths || !d_q || !d_k_slab || !d_v_slab || !d_out)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null batched-decode operand");
  // Pack the per-sequence tables into CSR (the reference passes pointer
  // arrays, which cannot cross the device boundary).
  std::vector<int32_t> qlens(num_seqs, 1), offsets(num_seqs + 1, 0), ids;
  for (int64_t b = 0; b < num_seqs; ++b) {
    const int64_t L = h_lengths[b];
    if (L < 1 || L > (int64_t{1} << 30))
      return SetError(ctx, EHIP_INVALID_ARGUMENT, "lengths[%lld]=%lld out of range",
                      static_cast<long long>(b), static_cast<long long>(L));
    if (!h_block_tables[b])
      return SetError(ctx, EHIP_INVALID_ARGUMENT, "block_tables[%lld] is null",
                      static_cast<long long>(b));
    const int64_t need = (L + block_size - 1) / block_size;
    ids.insert(ids.end(), h_block_tables[b], h_block_tables[b] + need);
    if (ids.size() > static_cast<size_t>(INT32_MAX))
      return SetError(ctx, EHIP_INVALID_ARGUMENT, "too many table entries");
    offsets[b + 1] = static_cast<int32_t>(ids.size());
  }
  ehip_step_desc s{static_cast<int32_t>(num_seqs), 0, qlens.data(), h_lengths, offsets.data(),
                   ids.data(), nullptr};
  Plan plan;
  if (int rc = ehip::BuildPlan(g, s, ctx->tune, &plan, &err))
    return SetError(ctx, rc, "%s", err.c_str());
  if (int rc = UploadPlan(ctx, g, std::move(plan), nullptr)) return rc;
  return LaunchAttention(ctx, d_q, d_k_slab, d_v_slab, d_out);
}
}  // namespace

int ehip_paged_decode_attention_batched_f32(
    ehip_ctx* ctx, const float* d_q, const float* d_k_slab, const float* d_v_slab,
    const int32_t* const* h_block_tables, const int64_t* h_lengths, int64_t num_seqs,
    int64_t heads, int64_t kv_heads, int64_t d, int64_t block_size, int64_t block_stride,
    int64_t slab_blocks, float scale, float* d_out) {
  return BatchedDecode(ctx, EHIP_KV_F32, d_q, d_k_slab, d_v_slab, h_block_tables, h_lengths,
                       num_seqs, heads, kv_heads, d, block_size, block_stride, slab_blocks,
                       scale, d_out);
}

int ehip_paged_decode_attention_batched_bf16(
    ehip_ctx* ctx, const float* d_q, const uint16_t* d_k_slab, const uint16_t* d_v_slab,
    const int32_t* const* h_block_tables, const int64_t* h_lengths, int64_t num_seqs,
    int64_t heads, int64_t kv_heads, int64_t d, int64_t block_size, int64_t block_stride,
    int64_t slab_blocks, float scale, float* d_out) {
  return BatchedDecode(ctx, EHIP_KV_BF16, d_q, d_k_slab, d_v_slab, h_block_tables, h_lengths,
                       num_seqs, heads, kv_heads, d, block_size, block_stride, slab_blocks,
                       scale, d_out);
}

// ------------------------------------------------------------ step path --

namespace {
// Query rows per MFMA prefill item for the geometry (0: chunks stay on the
// decode kernels).
int StepPrefillRows(const ehip_geometry& g) {
  const int64_t stride = ehip::BlockStride(g);
  const int64_t slab_bytes = g.slab_blocks > 0 && stride > 0 &&
                                     g.slab_blocks <= INT64_MAX / stride / 2
                                 ? g.slab_blocks * stride * 2
                                 : INT64_MAX;
  return ehip::PrefillRowsPerItem(g.kv_dtype, g.head_dim,
                                  g.kv_heads > 0 ? g.heads / g.kv_heads : 0, g.block_size,
                                  slab_bytes);
}
}  // namespace

int ehip_step_upload(ehip_ctx* ctx, const ehip_geometry* geom, const ehip_step_desc* step) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!geom || !step) return SetError(ctx, EHIP_INVALID_ARGUMENT, "null geometry or step");
  Plan plan;
  std::string err;
  if (int rc = ehip::BuildPlan(*geom, *step, ctx->tune, &plan, &err, StepPrefillRows(*geom)))
    return SetError(ctx, rc, "%s", err.c_str());
  return UploadPlan(ctx, *geom, std::move(plan), nullptr);
}

int ehip_step_kv_append(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                        void* d_k_slab, void* d_v_slab) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ctx->have_step) return SetError(ctx, EHIP_FAILED_PRECONDITION, "no step uploaded");
  const Plan& plan = ctx->plan;
  if (plan.slots.empty()) {
    if (plan.rows.empty()) return EHIP_OK;
    return SetError(ctx, EHIP_FAILED_PRECONDITION, "the uploaded step has no slot mapping");
  }
  if (!d_src_k || !d_src_v || !d_k_slab || !d_v_slab)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null append operand");
  const ehip_geometry& g = ctx->geom;
  if (ehip::ScaledKv(g.kv_dtype))
    return SetError(ctx, EHIP_INVALID_ARGUMENT,
                    "INT8/FP8 slabs carry scales: use ehip_step_kv_append_int8 or _fp8");
  if (ehip::BlockStride(g) != int64_t{g.kv_heads} * g.block_size * g.head_dim)
    return SetError(ctx, EHIP_UNIMPLEMENTED, "append needs the dense Hkv*bs*d block stride");
  EHIP_HIP(ctx, ehip::LaunchKvScatter(d_src_k, d_src_v, ctx->d_slots,
                                      static_cast<int64_t>(plan.slots.size()), g.kv_heads,
                                      g.head_dim, g.block_size, g.slab_blocks, d_k_slab,
                                      d_v_slab, g.kv_dtype, ctx->d_err, ctx->stream));
  return EHIP_OK;
}

int ehip_step_rope_kv_append(ehip_ctx* ctx, float* d_q, const float* d_src_k,
                             const float* d_src_v, const float* d_cos, const float* d_sin,
                             int64_t table_positions, void* d_k_slab, void* d_v_slab) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ctx->have_step) return SetError(ctx, EHIP_FAILED_PRECONDITION, "no step uploaded");
  const Plan& plan = ctx->plan;
  if (plan.rows.empty()) return EHIP_OK;
  if (plan.slots.empty())
    return SetError(ctx, EHIP_FAILED_PRECONDITION, "the uploaded step has no slot mapping");
  if (!d_q || !d_src_k || !d_src_v || !d_cos || !d_sin || !d_k_slab || !d_v_slab)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null rope/append operand");
  const ehip_geometry& g = ctx->geom;
  if (ehip::ScaledKv(g.kv_dtype))
    return SetError(ctx, EHIP_UNIMPLEMENTED, "fused RoPE + append covers fp32 and bf16 slabs");
  if (g.head_dim % 2 != 0)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "RoPE needs an even head_dim (got %d)",
                    g.head_dim);
  if (plan.max_length > table_positions)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "position %lld outside the RoPE tables [0, %lld)",
                    static_cast<long long>(plan.max_length - 1),
                    static_cast<long long>(table_positions));
  if (ehip::BlockStride(g) != int64_t{g.kv_heads} * g.block_size * g.head_dim)
    return SetError(ctx, EHIP_UNIMPLEMENTED, "append needs the dense Hkv*bs*d block stride");
  EHIP_HIP(ctx, ehip::LaunchRopeKvAppend(d_q, d_src_k, d_src_v, ctx->d_rows, d_cos, d_sin,
                                         ctx->d_slots, static_cast<int64_t>(plan.rows.size()),
                                         g.heads, g.kv_heads, g.head_dim, g.block_size,
                                         g.slab_blocks, d_k_slab, d_v_slab, g.kv_dtype,
                                         ctx->d_err, ctx->stream));
  return EHIP_OK;
}

int ehip_step_attention(ehip_ctx* ctx, const float* d_q, const void* d_k_slab,
                        const void* d_v_slab, float* d_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ctx->have_step) return SetError(ctx, EHIP_FAILED_PRECONDITION, "no step uploaded");
  if (ctx->plan.rows.empty()) return EHIP_OK;
  if (!d_q || !d_k_slab || !d_v_slab || !d_out)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null attention operand");
  if (ehip::ScaledKv(ctx->geom.kv_dtype))
    return SetError(ctx, EHIP_INVALID_ARGUMENT,
                    "INT8/FP8 slabs carry scales: use ehip_step_attention_int8 or _fp8");
  return LaunchAttention(ctx, d_q, d_k_slab, d_v_slab, d_out);
}

int ehip_step_append_attention(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                               const float* d_q, void* d_k_slab, void* d_v_slab, float* d_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ctx->have_step) return SetError(ctx, EHIP_FAILED_PRECONDITION, "no step uploaded");
  const Plan& plan = ctx->plan;
  const ehip_geometry& g = ctx->geom;
  if (plan.rows.empty()) return EHIP_OK;
  if (plan.slots.empty())
    return SetError(ctx, EHIP_FAILED_PRECONDITION, "the uploaded step has no slot mapping");
  if (!d_src_k || !d_src_v || !d_q || !d_k_slab || !d_v_slab || !d_out)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null append/attention operand");
  if (ehip::ScaledKv(g.kv_dtype))
    return SetError(ctx, EHIP_INVALID_ARGUMENT,
                    "INT8/FP8 slabs carry scales: use the _int8 / _fp8 append and attention");
  if (ehip::BlockStride(g) != int64_t{g.kv_heads} * g.block_size * g.head_dim)
    return SetError(ctx, EHIP_UNIMPLEMENTED, "append needs the dense Hkv*bs*d block stride");
  // One launch (plus the split merge) when every row is a decode row on the
  // matrix-core kernel: the items ending at their rows' last keys append.
  if (ctx->tune.fused_append && plan.all_decode && !plan.items.empty() &&
      reinterpret_cast<uintptr_t>(d_src_k) % 8 == 0 && reinterpret_cast<uintptr_t>(d_src_v) % 8 == 0 &&
      ehip::DecodeMfmaCovers(StepDecodeParams(ctx, d_q, d_k_slab, d_v_slab, d_out), g.kv_dtype,
                             ctx->tune))
    return LaunchAttention(ctx, d_q, d_k_slab, d_v_slab, d_out, nullptr, nullptr, d_src_k,
                           d_src_v);
  EHIP_HIP(ctx, ehip::LaunchKvScatter(d_src_k, d_src_v, ctx->d_slots,
                                      static_cast<int64_t>(plan.slots.size()), g.kv_heads,
                                      g.head_dim, g.block_size, g.slab_blocks, d_k_slab, d_v_slab,
                                      g.kv_dtype, ctx->d_err, ctx->stream));
  return LaunchAttention(ctx, d_q, d_k_slab, d_v_slab, d_out);
}

namespace {

int ScaledAppend(ehip_ctx* ctx, int kv_dtype, const float* d_src_k, const float* d_src_v,
                 void* d_k_slab, void* d_v_slab, float* d_k_scale, float* d_v_scale) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ctx->have_step) return SetError(ctx, EHIP_FAILED_PRECONDITION, "no step uploaded");
  const Plan& plan = ctx->plan;
  const ehip_geometry& g = ctx->geom;
  if (g.kv_dtype != kv_dtype)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "the uploaded geometry is not %s KV",
                    kv_dtype == EHIP_KV_FP8 ? "FP8" : "INT8");
  if (plan.slots.empty()) {
    if (plan.rows.empty()) return EHIP_OK;
    return SetError(ctx, EHIP_FAILED_PRECONDITION, "the uploaded step has no slot mapping");
  }
  if (!d_src_k || !d_src_v || !d_k_slab || !d_v_slab || !d_k_scale || !d_v_scale)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null append operand");
  if (ehip::BlockStride(g) != int64_t{g.kv_heads} * g.block_size * g.head_dim)
    return SetError(ctx, EHIP_UNIMPLEMENTED, "append needs the dense Hkv*bs*d block stride");
  EHIP_HIP(ctx, ehip::LaunchAppendQ8(d_src_k, d_src_v, ctx->d_q8_groups,
                                     static_cast<int64_t>(plan.q8_groups.size()), ctx->d_q8_rows,
                                     g.kv_heads, g.head_dim, g.block_size, g.slab_blocks,
                                     d_k_slab, d_v_slab, d_k_scale, d_v_scale,
                                     kv_dtype == EHIP_KV_FP8, ctx->d_err, ctx->stream));
  return EHIP_OK;
}

int ScaledAttention(ehip_ctx* ctx, int kv_dtype, const float* d_q, const void* d_k_slab,
                    const void* d_v_slab, const float* d_k_scale, const float* d_v_scale,
                    float* d_out) {
  if (int rc = CheckCtx(ctx)) return rc;
  if (!ctx->have_step) return SetError(ctx, EHIP_FAILED_PRECONDITION, "no step uploaded");
  const ehip_geometry& g = ctx->geom;
  if (g.kv_dtype != kv_dtype)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "the uploaded geometry is not %s KV",
                    kv_dtype == EHIP_KV_FP8 ? "FP8" : "INT8");
  if (ctx->plan.rows.empty()) return EHIP_OK;
  if (!d_q || !d_k_slab || !d_v_slab || !d_k_scale || !d_v_scale || !d_out)
    return SetError(ctx, EHIP_INVALID_ARGUMENT, "null attention operand");
  if (g.slab_blocks * g.kv_heads >= (int64_t{1} << 29))
    return SetError(ctx, EHIP_UNIMPLEMENTED, "scale arrays above 2 GiB");
  return LaunchAttention(ctx, d_q, d_k_slab, d_v_slab, d_out, d_k_scale, d_v_scale);
}

}  // namespace

int ehip_step_kv_append_int8(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                             void* d_k_slab, void* d_v_slab, float* d_k_scale, float* d_v_scale) {
  return ScaledAppend(ctx, EHIP_KV_INT8, d_src_k, d_src_v, d_k_slab, d_v_slab, d_k_scale,
                      d_v_scale);
}

int ehip_step_attention_int8(ehip_ctx* ctx, const float* d_q, const void* d_k_slab,
                             const void* d_v_slab, const float* d_k_scale,
                             const float* d_v_scale, float* d_out) {
  return ScaledAttention(ctx, EHIP_KV_INT8, d_q, d_k_slab, d_v_slab, d_k_scale, d_v_scale, d_out);
}

int ehip_step_kv_append_fp8(ehip_ctx* ctx, const float* d_src_k, const float* d_src_v,
                            void* d_k_slab, void* d_v_slab, float* d_k_scale, float* d_v_scale) {
  return ScaledAppend(ctx, EHIP_KV_FP8, d_src_k, d_src_v, d_k_slab, d_v_slab, d_k_scale,
                      d_v_scale);
}

int ehip_step_attention_fp8(ehip_ctx* ctx, const float* d_q, const void* d_k_slab,
                            const void* d_v_slab, const float* d_k_scale, const float* d_v_scale,
                            float* d_out) {
  return ScaledAttention(ctx, EHIP_KV_FP8, d_q, d_k_slab, d_v_slab, d_k_scale, d_v_scale, d_out);
}

int ehip_step_info(const ehip_ctx* ctx, int64_t* rows, int64_t* items, int64_t* partials) {
  if (!ctx || !ctx->have_step) return EHIP_FAILED_PRECONDITION;
  if (rows) *rows = static_cast<int64_t>(ctx->plan.rows.size());
  if (items) *items = static_cast<int64_t>(ctx->plan.items.size() + ctx->plan.prefill.size());
  if (partials) *partials = ctx->plan.partials;
  return EHIP_OK;
}

int ehip_plan_counts(const ehip_geometry* geom, const ehip_step_desc* step, int64_t* rows,
                     int64_t* items, int64_t* partials, int32_t* split_tokens,
                     int64_t* joint_items, int64_t* shared_tokens) {
  if (!geom || !step) return EHIP_INVALID_ARGUMENT;
  Plan plan;
  std::string err;
  if (int rc = ehip::BuildPlan(*geom, *step, ehip::ReadTuning(), &plan, &err)) return rc;
  if (rows) *rows = static_cast<int64_t>(plan.rows.size());
  if (items) *items = static_cast<int64_t>(plan.items.size());
  if (partials) *partials = plan.partials;
  if (split_tokens) *split_tokens = plan.split_tokens;
  if (joint_items) *joint_items = plan.joint_items;
  if (shared_tokens) *shared_tokens = plan.shared_tokens;
  return EHIP_OK;
}

int ehip_plan_items(const ehip_geometry* geom, const ehip_step_desc* step, int32_t* out,
                    int64_t cap, int64_t* n) {
  if (!geom || !step || !n || cap < 0 || (cap > 0 && !out)) return EHIP_INVALID_ARGUMENT;
  Plan plan;
  std::string err;
  if (int rc = ehip::BuildPlan(*geom, *step, ehip::ReadTuning(), &plan, &err)) return rc;
  *n = static_cast<int64_t>(plan.items.size());
  const int64_t m = std::min<int64_t>(cap, *n);
  for (int64_t i = 0; i < m; ++i) {
    const ehip::WorkItem& w = plan.items[static_cast<size_t>(i)];
    int32_t* o = out + 8 * i;
    const bool x = !plan.items_x.empty();
    o[0] = w.row0;
    o[1] = w.row1;
    o[2] = x ? plan.items_x[static_cast<size_t>(i)].row2 : -1;
    o[3] = x ? plan.items_x[static_cast<size_t>(i)].row3 : -1;
    o[4] = w.tok_begin;
    o[5] = w.tok_end;
    o[6] = ehip::UnpackHk(w.hk_split);
    o[7] = ehip::UnpackSplit(w.hk_split);
  }
  return EHIP_OK;
}

int ehip_plan_prefill_items(const ehip_geometry* geom, const ehip_step_desc* step, int32_t* out,
                            int64_t cap, int64_t* n) {
  if (!geom || !step || !n || cap < 0 || (cap > 0 && !out)) return EHIP_INVALID_ARGUMENT;
  Plan plan;
  std::string err;
  if (int rc = ehip::BuildPlan(*geom, *step, ehip::ReadTuning(), &plan, &err,
                               StepPrefillRows(*geom)))
    return rc;
  *n = static_cast<int64_t>(plan.prefill.size());
  const int64_t m = std::min<int64_t>(cap, *n);
  for (int64_t i = 0; i < m; ++i) {
    const ehip::PrefillItem& w = plan.prefill[static_cast<size_t>(i)];
    int32_t* o = out + 9 * i;
    o[0] = w.row_base;
    o[1] = w.chunk;
    o[2] = w.past;
    o[3] = w.q0;
    o[4] = ehip::UnpackHk(w.hk_split);
    o[5] = ehip::UnpackSplit(w.hk_split);
    o[6] = w.key_begin;
    o[7] = w.key_end;
    o[8] = plan.rows[static_cast<size_t>(w.row_base + w.q0)].nsplit;
  }
  return EHIP_OK;
}

}  // extern "C"
