#include "plan.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <climits>
#include <cstdlib>
#include <cstring>
#include <utility>

namespace ehip {
namespace {

constexpr int32_t kTile = 64;             // split lengths are whole 64-key units
// About one work item per resident decode wavefront (2048 on MI355X) before
// the per-item length cap: each item pays its descriptor, query and
// first-tile round trips plus a partial slot, and the queue balances the
// rest (with 32 item sub-queues, 2048 measured faster than 4096 on C3,
// 150 -> 141 us, and C5, 268 -> 262 us; C4's items are all at the cap).
constexpr int64_t kTargetItems = 2048;
constexpr int32_t kMinSplit = 128;
// Steps this small (fewer than 128 items of kMinSplit keys) are latency-bound:
// each wavefront's walk over its range sets the time, so they split into
// single 64-key units (C1, 513 keys x 2 kv heads: 14 us against 17.5 us per
// attention call; C2, 500 items of 128 keys, is faster as it is).
constexpr int64_t kSmallStepUnits = int64_t{128} * kMinSplit;
constexpr int32_t kMaxSplitsPerRow = 64;  // bounds the merge a single wave performs
// Large steps (one item per resident wavefront would already mean ranges of
// at least kLargeStep keys) take ranges of kLargeMin..kLargeMax keys. Measured
// on MI355X (attention call per layer, one process, interleaved calls):
//   C4 (4.9M kv-head-keys):  1024: 397.0  1280: 393.7  1536: 389.0  2048: 408.8 us
//   C5 (2.9M):               1024: 279.5  1408: 262.3  1792: 275.5  2048: 274.8 us
//   C3 (1.1M decode, + the prefill chunks): 576: 151.6  768: 148.4  1024: 143.4
//                            1536: 156.7  2048: 184.7 us
// Fewer, longer items carry fewer startups and partials; past ~1536 keys the
// last items' walks set the tail.
constexpr int64_t kLargeStep = 512;
constexpr int64_t kLargeMin = 1024;
constexpr int64_t kLargeMax = 1536;

int Fail(std::string* err, int code, const char* fmt, long long a = 0, long long b = 0,
         long long c = 0) {
  char buf[256];
  std::snprintf(buf, sizeof(buf), fmt, a, b, c);
  if (err) *err = buf;
  return code;
}

int64_t RoundUp(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

}  // namespace

Tuning ReadTuning() {
  Tuning t;
  auto flag = [](const char* name, char off) {
    const char* v = std::getenv(name);
    return !(v && v[0] == off);
  };
  if (const char* v = std::getenv("EHIP_SPLIT_TOKENS")) {
    const long x = std::strtol(v, nullptr, 10);
    if (x > 0) t.split_tokens = static_cast<int32_t>(std::min<long>(x, INT32_MAX / 2));
  }
  if (const char* v = std::getenv("EHIP_TARGET_ITEMS")) {
    const long x = std::strtol(v, nullptr, 10);
    if (x > 0) t.target_items = x;
  }
  if (const char* v = std::getenv("EHIP_TAIL_SPLIT")) {
    const long x = std::strtol(v, nullptr, 10);
    if (x >= 0) t.tail_split = static_cast<int32_t>(std::min<long>(x, INT32_MAX / 2));
  }
  if (const char* v = std::getenv("EHIP_TAIL_FRAC")) {
    const double x = std::strtod(v, nullptr);
    if (x >= 0 && x <= 1) t.tail_frac = x;
  }
  if (const char* v = std::getenv("EHIP_SPLIT_EVEN")) t.split_even = v[0] == '1' ? 1 : v[0] == '0' ? 0 : -1;
  t.joint = flag("EHIP_NO_JOINT", '1');
  t.prefill = flag("EHIP_PREFILL", '0');
  if (const char* v = std::getenv("EHIP_PREFILL_SPLIT")) t.prefill_split = std::strtod(v, nullptr);
  if (const char* v = std::getenv("EHIP_DECODE_KERNEL")) t.decode_valu = std::strcmp(v, "valu") == 0;
  if (const char* v = std::getenv("EHIP_DECODE_TILE")) t.decode_tile16 = std::strcmp(v, "16") == 0;
  if (const char* v = std::getenv("EHIP_DECODE_BUFS")) t.decode_bufs3 = std::strcmp(v, "3") == 0;
  t.decode_persist = flag("EHIP_DECODE_PERSIST", '0');
  if (const char* v = std::getenv("EHIP_DECODE_SLOTS")) {
    const long x = std::strtol(v, nullptr, 10);
    if (x > 0) t.decode_slots = static_cast<int32_t>(std::min<long>(x, INT32_MAX));
  }
  t.decode_wg = flag("EHIP_DECODE_WG", '0');
  t.decode_split4 = flag("EHIP_DECODE_SPLIT4", '0');
  t.decode_qspread = flag("EHIP_DECODE_QSPREAD", '0');
  if (const char* v = std::getenv("EHIP_DECODE_QUEUES")) {
    const long x = std::strtol(v, nullptr, 10);
    if (x > 0) t.decode_queues = static_cast<int32_t>(std::min<long>(x, 1 << 20));
  }
  t.fused_append = flag("EHIP_FUSED_APPEND", '0');
  return t;
}

int64_t BlockStride(const ehip_geometry& g) {
  return g.block_stride != 0 ? g.block_stride
                             : int64_t{g.kv_heads} * g.block_size * g.head_dim;
}

int ValidateGeometry(const ehip_geometry& g, std::string* err) {
  if (g.heads < 1 || g.kv_heads < 1 || g.head_dim < 1)
    return Fail(err, EHIP_INVALID_ARGUMENT, "heads=%lld kv_heads=%lld d=%lld must be >= 1",
                g.heads, g.kv_heads, g.head_dim);
  if (g.heads % g.kv_heads != 0)
    return Fail(err, EHIP_INVALID_ARGUMENT, "heads=%lld is not a multiple of kv_heads=%lld",
                g.heads, g.kv_heads);
  if (g.head_dim > 256)
    return Fail(err, EHIP_UNIMPLEMENTED, "head_dim=%lld > 256 is not supported", g.head_dim);
  if (g.heads / g.kv_heads > 64)
    return Fail(err, EHIP_UNIMPLEMENTED, "GQA group %lld > 64 is not supported",
                g.heads / g.kv_heads);
  // The reference CHECKs bs | 64 (src/kernels/paged_attention.cpp:88-91) and the
  // pool admits {8,16,32,64} (src/kvcache/block_pool.cpp:28-31).
  if (g.block_size != 8 && g.block_size != 16 && g.block_size != 32 && g.block_size != 64)
    return Fail(err, EHIP_INVALID_ARGUMENT,
                "block_size=%lld must be one of 8, 16, 32, 64 (a power of two dividing 64)",
                g.block_size);
  if (g.kv_dtype != EHIP_KV_F32 && g.kv_dtype != EHIP_KV_BF16 && !ScaledKv(g.kv_dtype))
    return Fail(err, EHIP_INVALID_ARGUMENT,
                "kv_dtype=%lld is not F32 (0), BF16 (1), INT8 (2) or FP8 (3)", g.kv_dtype);
  if (ScaledKv(g.kv_dtype)) {
    // The scaled-KV kernels (MFMA QK^T over 16-token halves) cover these shapes.
    const int64_t grp = g.heads / g.kv_heads;
    if ((g.head_dim != 64 && g.head_dim != 128) ||
        (grp != 1 && grp != 2 && grp != 4 && grp != 8) || g.block_size < 16)
      return Fail(err, EHIP_UNIMPLEMENTED,
                  "INT8/FP8 KV needs head_dim 64 or 128, g in {1,2,4,8} and block_size >= 16 "
                  "(got d=%lld, g=%lld, bs=%lld)",
                  g.head_dim, grp, g.block_size);
  }
  if (g.reserved != 0) return Fail(err, EHIP_INVALID_ARGUMENT, "reserved field must be 0");
  if (g.slab_blocks < 1)
    return Fail(err, EHIP_INVALID_ARGUMENT, "slab_blocks=%lld must be >= 1", g.slab_blocks);
  const int64_t tile = int64_t{g.kv_heads} * g.block_size * g.head_dim;
  if (g.block_stride != 0 && g.block_stride < tile)
    return Fail(err, EHIP_INVALID_ARGUMENT, "block_stride=%lld < Hkv*bs*d=%lld",
                g.block_stride, tile);
  if (!std::isfinite(g.scale))
    return Fail(err, EHIP_INVALID_ARGUMENT, "scale must be finite");
  return EHIP_OK;
}

int32_t MaxSplitTokens(const ehip_geometry& g) {
  // A work item's table slice sits in the wavefront's lanes, two block ids
  // per lane: 128 blocks.
  return 128 * g.block_size;
}

static int64_t DecodeItemTarget(const ehip_geometry& g, const Tuning& tune) {
  if (tune.target_items > 0) return tune.target_items;
  return ScaledKv(g.kv_dtype) ? kTargetItems / 2 : kTargetItems;
}

int32_t ChooseSplitTokens(const ehip_geometry& g, int64_t unit_tokens, const Tuning& tune) {
  const int32_t max_split = MaxSplitTokens(g);
  if (tune.split_tokens > 0)
    return static_cast<int32_t>(std::min<int64_t>(RoundUp(tune.split_tokens, kTile), max_split));
  const int64_t target = DecodeItemTarget(g, tune);
  int64_t s = (unit_tokens + target - 1) / target;
  if (!ScaledKv(g.kv_dtype) && s >= kLargeStep) s = std::clamp(s, kLargeMin, kLargeMax);
  s = RoundUp(std::max<int64_t>(s, unit_tokens < kSmallStepUnits ? kTile : kMinSplit), kTile);
  return static_cast<int32_t>(std::min<int64_t>(s, max_split));
}

int32_t RowSplitTokens(const ehip_geometry& g, int32_t base, int32_t len) {
  int32_t sl = base;
  if ((len + sl - 1) / sl > kMaxSplitsPerRow) {
    const int64_t want = RoundUp((len + kMaxSplitsPerRow - 1) / kMaxSplitsPerRow, kTile);
    sl = static_cast<int32_t>(std::min<int64_t>(want, MaxSplitTokens(g)));
  }
  return sl;
}

int32_t SingleRowSplitTokens(const ehip_geometry& g, int64_t length, const Tuning& tune) {
  const int32_t base = ChooseSplitTokens(g, length * g.kv_heads, tune);
  return RowSplitTokens(g, base, static_cast<int32_t>(length));
}

namespace {

constexpr int32_t kMinJointTokens = 128;  // shorter shared runs are not worth a joint pass

// Full leading blocks two rows read from the same physical block ids, short
// of each row's last key: a row whose length is a multiple of bs keeps its
// last block for a range of its own, so every row has a non-joint range
// ending at its last key (the item that appends the row's new token in the
// fused append + attention launch).
int32_t SharedFullBlocks(const Plan& plan, const RowDesc& a, const RowDesc& b, int32_t bs) {
  const int32_t limit = (std::min(a.length, b.length) - 1) / bs;
  if (a.table_off == b.table_off) return limit;  // rows of one sequence
  const int32_t* ta = plan.table_ids.data() + a.table_off;
  const int32_t* tb = plan.table_ids.data() + b.table_off;
  int32_t c = 0;
  while (c < limit && ta[c] == tb[c]) ++c;
  return c;
}

// One key range of a row, or of a joint group's rows over their shared
// prefix (rows[1..] = -1 where absent).
struct KeyRange {
  int32_t rows[kMaxJointRows];
  int32_t tb, te;
  bool joint() const { return rows[1] >= 0; }
};

// Piece length for cutting `keys` keys into ranges of at most sl keys, evened
// out: the same number of pieces, of whole kTile units, the last one the
// shortest (a run of 1.1 sl keys makes two pieces of ~0.55 sl instead of
// sl + 0.1 sl).
int32_t EvenStep(int32_t sl, int32_t keys) {
  if (keys <= sl) return sl;
  const int32_t pieces = (keys + sl - 1) / sl;
  return static_cast<int32_t>(
      std::min<int64_t>(sl, RoundUp((keys + pieces - 1) / pieces, kTile)));
}

// Tail pieces. When a step has more items than the queue hands out first,
// the queue's last items set the launch's end: a wavefront streams ~3 GB/s
// (a 1024-key bf16 range of d = 128 takes ~170 us), and on C4 the items that
// started in the last 120 us were up to 648 keys long, ~8% of the step's
// keys. The smallest single-row ranges, up to Tuning::tail_frac of the
// step's keys (times rows), are cut into pieces of Tuning::tail_split keys;
// ordered costliest first, the pieces are the queue's last items. A row keeps
// at most kMaxSplitsPerRow ranges. Off by default: every extra item costs its
// wavefront ~8 us of startup, more than the shorter tail saves (C4 attention
// call, 100 interleaved calls each: 398.8 us without pieces, 404.9 / 407.9 /
// 413.8 us with 128-key pieces over 5 / 8 / 12% of the keys).
void CutTail(const ehip_geometry& g, const Tuning& tune, const std::vector<RowDesc>& rows,
             std::vector<KeyRange>* ranges) {
  const int32_t ts = static_cast<int32_t>(RoundUp(tune.tail_split, kTile));
  const int64_t target = tune.target_items > 0 ? tune.target_items : kTargetItems;
  if (ts <= 0 || tune.tail_frac <= 0 ||
      static_cast<int64_t>(ranges->size()) * g.kv_heads <= target)
    return;
  std::vector<KeyRange>& rg = *ranges;
  int64_t total = 0;
  std::vector<int32_t> count(rows.size(), 0);
  std::vector<size_t> cand;
  for (size_t i = 0; i < rg.size(); ++i) {
    int rws = 0;
    for (int32_t r : rg[i].rows)
      if (r >= 0) {
        ++rws;
        ++count[r];
      }
    total += int64_t{rg[i].te - rg[i].tb} * rws;
    if (!rg[i].joint() && rg[i].te - rg[i].tb > ts) cand.push_back(i);
  }
  std::stable_sort(cand.begin(), cand.end(), [&](size_t a, size_t b) {
    return rg[a].te - rg[a].tb < rg[b].te - rg[b].tb;
  });
  const double budget = tune.tail_frac * static_cast<double>(total);
  int64_t acc = 0;
  std::vector<char> cut(rg.size(), 0);
  for (size_t i : cand) {
    const int32_t len = rg[i].te - rg[i].tb;
    if (static_cast<double>(acc + len) > budget) break;
    const int32_t r = rg[i].rows[0];
    const int32_t extra = (len + ts - 1) / ts - 1;
    if (count[r] + extra > kMaxSplitsPerRow) continue;
    count[r] += extra;
    acc += len;
    cut[i] = 1;
  }
  std::vector<KeyRange> out;
  out.reserve(rg.size() + static_cast<size_t>(acc / ts) + 1);
  for (size_t i = 0; i < rg.size(); ++i) {
    if (!cut[i]) {
      out.push_back(rg[i]);
      continue;
    }
    for (int32_t t = rg[i].tb; t < rg[i].te; t += ts) {
      KeyRange kr = rg[i];
      kr.tb = t;
      kr.te = std::min(rg[i].te, t + ts);
      out.push_back(kr);
    }
  }
  rg.swap(out);
}

// Groups rows that share leading blocks (greedy over rows ordered by their
// first block id and table), splits every row into whole-tile key ranges
// (joint ranges first), assigns partial slots and orders the work longest
// first.
// skip[r] > 0: row r is served by the prefill kernel in skip[r] key splits.
void FinishPlan(const ehip_geometry& g, const Tuning& tune, Plan* plan, bool allow_joint,
                const std::vector<int32_t>* skip = nullptr) {
  const int32_t bs = g.block_size;
  const size_t n = plan->rows.size();
  auto skipped = [&](size_t r) { return skip && (*skip)[r] > 0; };
  int64_t units = 0;
  for (size_t r = 0; r < n; ++r)
    if (!skipped(r)) units += int64_t{plan->rows[r].length} * g.kv_heads;
  const int32_t base = ChooseSplitTokens(g, units, tune);
  plan->split_tokens = base;
  plan->groups.clear();
  plan->group_start.assign(1, 0);
  plan->joint_items = 0;
  plan->joint_rows = 1;
  plan->shared_tokens = 0;

  std::vector<int32_t> joint_len(n, 0);
  const int cap = JointRowsCap(g.heads / g.kv_heads);
  if (allow_joint && tune.joint && cap >= 2 && n >= 2) {
    std::vector<int32_t> order;
    order.reserve(n);
    for (size_t i = 0; i < n; ++i)
      if (!skipped(i)) order.push_back(static_cast<int32_t>(i));
    auto first_block = [&](int32_t r) { return plan->table_ids[plan->rows[r].table_off]; };
    std::sort(order.begin(), order.end(), [&](int32_t a, int32_t b) {
      const int32_t fa = first_block(a), fb = first_block(b);
      if (fa != fb) return fa < fb;
      if (plan->rows[a].table_off != plan->rows[b].table_off)
        return plan->rows[a].table_off < plan->rows[b].table_off;
      return a < b;
    });
    // A group starts at a row and takes the following rows while that saves
    // more re-read keys: with m members and common prefix C (full blocks), a
    // member sharing c blocks with the first row makes the common prefix
    // C' = min(C, c), and it joins if m * C' > (m - 1) * C (and C' spans at
    // least kMinJointTokens keys).
    for (size_t i = 0; i + 1 < order.size();) {
      const int32_t a = order[i];
      int32_t common = INT32_MAX;
      size_t j = i + 1;
      for (; j < order.size() && static_cast<int>(j - i) < cap; ++j) {
        const int32_t c = std::min(common, SharedFullBlocks(*plan, plan->rows[a],
                                                            plan->rows[order[j]], bs));
        const int64_t m = static_cast<int64_t>(j - i);  // members before order[j] joins
        if (c * bs < kMinJointTokens) break;
        if (common != INT32_MAX && m * int64_t{c} <= (m - 1) * int64_t{common}) break;
        common = c;
      }
      if (j - i < 2) {
        ++i;
        continue;
      }
      for (size_t k = i; k < j; ++k) {
        plan->groups.push_back(order[k]);
        joint_len[order[k]] = common * bs;
      }
      plan->group_start.push_back(static_cast<int32_t>(plan->groups.size()));
      plan->shared_tokens += int64_t{common} * bs * static_cast<int64_t>(j - i - 1);
      plan->joint_rows = std::max(plan->joint_rows, static_cast<int32_t>(j - i));
      i = j;
    }
  }
  const size_t n_groups = plan->group_start.size() - 1;
  auto members = [&](size_t k) {
    return std::pair<const int32_t*, const int32_t*>(plan->groups.data() + plan->group_start[k],
                                                     plan->groups.data() + plan->group_start[k + 1]);
  };

  // Split length per row (a group's members use the largest of theirs).
  std::vector<int32_t> split_len(n);
  for (size_t r = 0; r < n; ++r) split_len[r] = RowSplitTokens(g, base, plan->rows[r].length);
  for (size_t k = 0; k < n_groups; ++k) {
    const auto [b, e] = members(k);
    int32_t sl = 0;
    for (const int32_t* r = b; r != e; ++r) sl = std::max(sl, split_len[*r]);
    for (const int32_t* r = b; r != e; ++r) split_len[*r] = sl;
  }

  // Key ranges: a group's shared prefix [0, P) in joint ranges, then each
  // row's own keys [P, L), in pieces of the row's split length. Every range
  // becomes one work item per kv head. When every item gets a wavefront of
  // its own (no more items than the decode target), the pieces of each run
  // are evened out (same count): C3's 1256 decode items, attention call
  // 135.2 against 138.0 us (three interleaved pairs of contexts). With more
  // items than that the queue hands out the short last pieces of fixed-length
  // cuts last, which balances better: even cuts took C4 from 385.4 to 398.9 us
  // and C5 from 262.3 to 295.8 us.
  std::vector<KeyRange> ranges;
  auto cut_ranges = [&](bool even) {
    ranges.clear();
    for (size_t k = 0; k < n_groups; ++k) {
      const auto [b, e] = members(k);
      const int32_t P = joint_len[*b];
      const int32_t sl = even ? EvenStep(split_len[*b], P) : split_len[*b];
      for (int32_t t = 0; t < P; t += sl) {
        KeyRange kr{{-1, -1, -1, -1}, t, std::min(P, t + sl)};
        std::copy(b, e, kr.rows);
        ranges.push_back(kr);
      }
    }
    for (size_t r = 0; r < n; ++r) {
      if (skipped(r)) continue;
      const int32_t L = plan->rows[r].length;
      const int32_t sl = even ? EvenStep(split_len[r], L - joint_len[r]) : split_len[r];
      for (int32_t t = joint_len[r]; t < L; t += sl)
        ranges.push_back(KeyRange{{static_cast<int32_t>(r), -1, -1, -1}, t, std::min(L, t + sl)});
    }
  };
  cut_ranges(tune.split_even > 0);
  if (tune.split_even < 0 &&
      static_cast<int64_t>(ranges.size()) * g.kv_heads <= DecodeItemTarget(g, tune))
    cut_ranges(true);
  CutTail(g, tune, plan->rows, &ranges);

  // Split indices follow key order within a row. Joint ranges cover the
  // leading keys of every member, so numbering them first (in key order)
  // gives all members the same index for each.
  std::stable_sort(ranges.begin(), ranges.end(), [](const KeyRange& x, const KeyRange& y) {
    if (x.joint() != y.joint()) return x.joint();
    return x.rows[0] != y.rows[0] ? x.rows[0] < y.rows[0] : x.tb < y.tb;
  });
  size_t n_joint_ranges = 0;
  while (n_joint_ranges < ranges.size() && ranges[n_joint_ranges].joint()) ++n_joint_ranges;
  std::vector<int32_t> nsplit(n, 0), split_of(ranges.size());
  for (size_t i = 0; i < ranges.size(); ++i) {
    split_of[i] = nsplit[ranges[i].rows[0]];
    for (int32_t r : ranges[i].rows)
      if (r >= 0) ++nsplit[r];
  }
  int64_t split_base = 0;
  plan->any_split = false;
  plan->merge_rows.clear();
  for (size_t r = 0; r < n; ++r) {
    RowDesc& rd = plan->rows[r];
    rd.nsplit = skipped(r) ? ((*skip)[r] > 1 ? (*skip)[r] : 0) : nsplit[r];
    rd.split_base = static_cast<int32_t>(split_base);
    split_base += rd.nsplit;
    plan->any_split = plan->any_split || rd.nsplit > 1;
    if (rd.nsplit > 1) plan->merge_rows.push_back(static_cast<int32_t>(r));
  }
  plan->partials = split_base * g.kv_heads;
  for (size_t r = 0; r < n; ++r)
    if (plan->rows[r].nsplit >= (1 << kSplitBits)) plan->partials = -1;  // rejected by BuildPlan

  plan->items.clear();
  plan->items_x.clear();
  struct Entry {
    WorkItem w;
    ItemRowsX x;
  };
  std::vector<Entry> entries;
  entries.reserve(ranges.size() * g.kv_heads);
  for (size_t i = 0; i < ranges.size(); ++i) {
    const KeyRange& kr = ranges[i];
    const bool last = !kr.joint() && kr.te == plan->rows[kr.rows[0]].length;
    for (int32_t hk = 0; hk < g.kv_heads; ++hk)
      entries.push_back(Entry{WorkItem{kr.rows[0], kr.rows[1], kr.tb, kr.te,
                                       PackHkSplit(hk, split_of[i]) | (last ? kLastRangeFlag : 0),
                                       plan->rows[kr.rows[0]].table_off, 0, 0, 0, 0},
                              ItemRowsX{kr.rows[2], kr.rows[3]}});
  }
  plan->joint_items = static_cast<int64_t>(n_joint_ranges) * g.kv_heads;
  // Costliest first, so the tail of the dispatch is short items. A joint
  // item reads its keys once but does the arithmetic of both rows; counting
  // it as its keys times its rows starts the joint items with the first
  // wave of the queue instead of behind every full-length single-row item
  // (C4: 440 -> 428 us per launch on MI355X; weights 1.5 to 3 measured
  // alike, 1 left the joint items in the tail).
  auto cost = [](const Entry& e) {
    const int rows = 1 + (e.w.row1 >= 0) + (e.x.row2 >= 0) + (e.x.row3 >= 0);
    return int64_t{e.w.tok_end - e.w.tok_begin} * rows;
  };
  std::stable_sort(entries.begin(), entries.end(),
                   [&](const Entry& x, const Entry& y) { return cost(x) > cost(y); });
  plan->items.reserve(entries.size());
  for (const Entry& e : entries) plan->items.push_back(e.w);
  if (plan->joint_rows > 2) {
    plan->items_x.reserve(entries.size());
    for (const Entry& e : entries) plan->items_x.push_back(e.x);
  }
  // The block ids of each item's first four 16-token halves ride in the
  // item, so a wavefront issues its first two tiles' K/V loads at once
  // without waiting for its table slice (-1 when the table is
  // device-resident and unknown here).
  for (WorkItem& w : plan->items) {
    if (plan->table_ids.empty()) {
      w.first_block0 = w.first_block1 = w.first_block2 = w.first_block3 = -1;
      continue;
    }
    const int32_t* t = plan->table_ids.data() + w.table_off;
    auto at = [&](int32_t off) { return t[std::min(w.tok_begin + off, w.tok_end - 1) / g.block_size]; };
    w.first_block0 = at(0);
    w.first_block1 = at(16);
    w.first_block2 = at(32);
    w.first_block3 = at(48);
  }
}

}  // namespace

namespace {

// INT8/FP8 append groups: the step's rows grouped by destination block, each
// group's rows in offset order with consecutive offsets (tokens append in
// order; a block takes rows of one sequence only).
int BuildQ8Groups(const ehip_geometry& g, Plan* plan, std::string* err) {
  const int64_t n = static_cast<int64_t>(plan->slots.size());
  std::vector<int32_t> order(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) order[static_cast<size_t>(i)] = static_cast<int32_t>(i);
  std::stable_sort(order.begin(), order.end(),
                   [&](int32_t a, int32_t b) { return plan->slots[a] < plan->slots[b]; });
  for (int64_t i = 0; i < n;) {
    const int64_t block = plan->slots[order[i]] / g.block_size;
    const int64_t off0 = plan->slots[order[i]] % g.block_size;
    int64_t j = i;
    while (j < n && plan->slots[order[j]] / g.block_size == block) {
      if (plan->slots[order[j]] % g.block_size != off0 + (j - i))
        return Fail(err, EHIP_INVALID_ARGUMENT,
                    "scaled-KV append: rows landing in block %lld do not take consecutive slots "
                    "(slot %lld)",
                    block, plan->slots[order[j]]);
      ++j;
    }
    plan->q8_groups.push_back(Q8Group{static_cast<int32_t>(block), static_cast<int32_t>(off0),
                                      static_cast<int32_t>(j - i),
                                      static_cast<int32_t>(plan->q8_rows.size())});
    for (int64_t k = i; k < j; ++k) plan->q8_rows.push_back(order[k]);
    i = j;
  }
  return EHIP_OK;
}

}  // namespace

int BuildPlan(const ehip_geometry& g, const ehip_step_desc& s, const Tuning& tune, Plan* plan,
              std::string* err, int prefill_rows, bool head_major) {
  ehip_geometry checked = g;
  if (head_major) {
    if (g.block_stride != int64_t{g.block_size} * g.head_dim)
      return Fail(err, EHIP_INVALID_ARGUMENT, "a head-major cache has block_stride = bs * d");
    checked.block_stride = 0;
  }
  if (int rc = ValidateGeometry(checked, err)) return rc;
  if (s.num_seqs < 0) return Fail(err, EHIP_INVALID_ARGUMENT, "num_seqs=%lld < 0", s.num_seqs);
  if (s.reserved != 0) return Fail(err, EHIP_INVALID_ARGUMENT, "reserved field must be 0");
  plan->rows.clear();
  plan->items.clear();
  plan->prefill.clear();
  plan->table_ids.clear();
  plan->slots.clear();
  plan->q8_groups.clear();
  plan->q8_rows.clear();
  plan->partials = 0;
  plan->max_length = 0;
  const int32_t B = s.num_seqs;
  if (B == 0) {
    FinishPlan(g, tune, plan, false);
    return EHIP_OK;
  }
  if (!s.h_query_lens || !s.h_context_lens || !s.h_table_offsets || !s.h_table_ids)
    return Fail(err, EHIP_INVALID_ARGUMENT, "step arrays must be non-null");
  if (s.h_table_offsets[0] != 0)
    return Fail(err, EHIP_INVALID_ARGUMENT, "table_offsets[0]=%lld must be 0",
                s.h_table_offsets[0]);
  int64_t total_rows = 0;
  for (int32_t b = 0; b < B; ++b) {
    const int64_t T = s.h_query_lens[b];
    const int64_t L = s.h_context_lens[b];
    if (T < 1) return Fail(err, EHIP_INVALID_ARGUMENT, "query_lens[%lld]=%lld < 1", b, T);
    if (L < T || L > (int64_t{1} << 30))
      return Fail(err, EHIP_INVALID_ARGUMENT, "context_lens[%lld]=%lld out of range (T=%lld)",
                  b, L, T);
    const int64_t lo = s.h_table_offsets[b], hi = s.h_table_offsets[b + 1];
    const int64_t need = (L + g.block_size - 1) / g.block_size;
    if (hi < lo || hi - lo < need)
      return Fail(err, EHIP_INVALID_ARGUMENT,
                  "sequence %lld: table has %lld entries, needs ceil(L/bs)=%lld", b, hi - lo,
                  need);
    for (int64_t i = lo; i < lo + need; ++i) {
      const int32_t id = s.h_table_ids[i];
      if (id < 0 || id >= g.slab_blocks)
        return Fail(err, EHIP_INVALID_ARGUMENT, "sequence %lld: block id %lld outside [0, %lld)",
                    b, id, g.slab_blocks);
    }
    total_rows += T;
  }
  const int64_t n_ids = s.h_table_offsets[B];
  if (n_ids > (int64_t{1} << 31) - 1 || total_rows > (int64_t{1} << 24))
    return Fail(err, EHIP_INVALID_ARGUMENT, "step too large (%lld ids, %lld rows)", n_ids,
                total_rows);
  plan->table_ids.assign(s.h_table_ids, s.h_table_ids + n_ids);
  plan->rows.reserve(total_rows);
  for (int32_t b = 0; b < B; ++b) {
    const int32_t T = s.h_query_lens[b];
    const int64_t L = s.h_context_lens[b];
    const int64_t P = L - T;
    for (int32_t t = 0; t < T; ++t)
      plan->rows.push_back(RowDesc{s.h_table_offsets[b], static_cast<int32_t>(P + t + 1), 0, 0});
    plan->max_length = std::max(plan->max_length, L);
  }
  if (s.h_slot_mapping) {
    const int64_t cap = g.slab_blocks * g.block_size;
    for (int64_t i = 0; i < total_rows; ++i) {
      const int64_t slot = s.h_slot_mapping[i];
      if (slot < 0 || slot >= cap)
        return Fail(err, EHIP_INVALID_ARGUMENT, "slot_mapping[%lld]=%lld outside [0, %lld)", i,
                    slot, cap);
    }
    plan->slots.assign(s.h_slot_mapping, s.h_slot_mapping + total_rows);
    if (ScaledKv(g.kv_dtype))
      if (int rc = BuildQ8Groups(g, plan, err)) return rc;
  }
  if (g.kv_heads >= (1 << kHkBits))
    return Fail(err, EHIP_UNIMPLEMENTED, "kv_heads=%lld >= 4096", g.kv_heads);

  // Chunks big enough for the MFMA prefill kernel leave the decode partition.
  std::vector<int32_t> skip(plan->rows.size(), 0);
  if (prefill_rows > 0 && tune.prefill) {
    struct Block { int32_t b, q0, keys; };
    std::vector<Block> blocks;
    std::vector<int32_t> row_base(B + 1, 0);
    for (int32_t b = 0; b < B; ++b) row_base[b + 1] = row_base[b] + s.h_query_lens[b];
    int64_t total_tiles = 0;
    for (int32_t b = 0; b < B; ++b) {
      const int32_t T = s.h_query_lens[b];
      if (T < kMinPrefillRows) continue;
      const int32_t P = static_cast<int32_t>(s.h_context_lens[b] - T);
      for (int32_t q0 = 0; q0 < T; q0 += prefill_rows) {
        blocks.push_back({b, q0, P + std::min(T, q0 + prefill_rows)});
        total_tiles += (blocks.back().keys + kPrefillTile - 1) / kPrefillTile;
      }
      std::fill(skip.begin() + row_base[b], skip.begin() + row_base[b + 1], 1);
    }
    // Key splits: a block with more than twice the per-workgroup share of
    // the step's tiles is cut into splits of about that share, so the last
    // query blocks of a long chunk do not walk all their keys alone
    // Tuning::prefill_split: 0 keeps every block whole; a number x > 0
    // splits blocks longer than x shares (default 2: on C3, x = 1 measured
    // 58.9 us per layer against 45.7 us, as the extra partials and merge cost
    // more than the shorter critical path saves; the C5 re-prefill is the
    // same either way).
    const double split_mult = tune.prefill_split;
    const bool split_ok = split_mult > 0.0;
    const int64_t share = std::max<int64_t>(
        kMinPrefillSplitTiles,
        (total_tiles * g.kv_heads + kPrefillSlots - 1) / kPrefillSlots);
    // Tiles per key split of a block. The split count a row records must be
    // the number of pieces actually cut: with the cap on splits, ceil(tiles /
    // per) can fall below the count asked for (e.g. 626 tiles asked in 64
    // pieces take 10 tiles each, i.e. 63 pieces), and a recorded count above
    // it would make the merge read partial slots nothing wrote.
    auto block_tiles_per_split = [&](const Block& bl) {
      const int64_t tiles = (bl.keys + kPrefillTile - 1) / kPrefillTile;
      if (!split_ok || static_cast<double>(tiles) <= split_mult * static_cast<double>(share))
        return tiles;
      const int64_t want = std::min<int64_t>((tiles + share - 1) / share, kMaxSplitsPerRow);
      return (tiles + want - 1) / want;
    };
    // Most keys first; kv head fastest, so the blocks of one kv head are
    // dispatched 8 workgroups apart and land on one XCD's L2 together.
    std::stable_sort(blocks.begin(), blocks.end(),
                     [](const Block& x, const Block& y) { return x.keys > y.keys; });
    struct Piece { int32_t bi, split, kb, ke; };
    std::vector<Piece> pieces;
    for (size_t i = 0; i < blocks.size(); ++i) {
      const Block& bl = blocks[i];
      const int32_t T = s.h_query_lens[bl.b];
      const int32_t tiles = (bl.keys + kPrefillTile - 1) / kPrefillTile;
      const int32_t per = static_cast<int32_t>(block_tiles_per_split(bl));
      const int32_t ns = (tiles + per - 1) / per;  // pieces cut below, one per split slot
      const int32_t r0 = row_base[bl.b] + bl.q0;
      const int32_t r1 = row_base[bl.b] + std::min(T, bl.q0 + prefill_rows);
      std::fill(skip.begin() + r0, skip.begin() + r1, ns);
      for (int32_t sp = 0, kb = 0; kb < bl.keys; ++sp, kb += per * kPrefillTile)
        pieces.push_back({static_cast<int32_t>(i), sp, kb,
                          std::min(bl.keys, kb + per * kPrefillTile)});
    }
    // Longest piece first (the sort above keeps blocks in key order).
    std::stable_sort(pieces.begin(), pieces.end(), [](const Piece& x, const Piece& y) {
      return x.ke - x.kb > y.ke - y.kb;
    });
    for (const Piece& pc : pieces) {
      const Block& bl = blocks[pc.bi];
      const int32_t T = s.h_query_lens[bl.b];
      const int32_t P = static_cast<int32_t>(s.h_context_lens[bl.b] - T);
      for (int32_t hk = 0; hk < g.kv_heads; ++hk)
        plan->prefill.push_back(PrefillItem{row_base[bl.b], T, P, bl.q0, PackHkSplit(hk, pc.split),
                                            s.h_table_offsets[bl.b], pc.kb, pc.ke});
    }
  }
  FinishPlan(g, tune, plan, true, &skip);
  if (plan->partials < 0)
    return Fail(err, EHIP_UNIMPLEMENTED, "a row needs %lld or more key splits",
                int64_t{1} << kSplitBits);
  plan->all_decode = static_cast<int64_t>(plan->rows.size()) == B && plan->prefill.empty();
  return EHIP_OK;
}

int BuildSingleRowPlan(const ehip_geometry& g, int64_t length, int64_t num_blocks,
                       const Tuning& tune, Plan* plan, std::string* err) {
  if (int rc = ValidateGeometry(g, err)) return rc;
  if (length < 1 || length > (int64_t{1} << 30))
    return Fail(err, EHIP_INVALID_ARGUMENT, "length=%lld out of range", length);
  if ((length + g.block_size - 1) / g.block_size > num_blocks)
    return Fail(err, EHIP_INVALID_ARGUMENT, "ceil(length/bs) exceeds num_blocks=%lld",
                num_blocks);
  plan->rows.assign(1, RowDesc{0, static_cast<int32_t>(length), 0, 0});
  plan->max_length = length;
  plan->table_ids.clear();
  plan->slots.clear();
  FinishPlan(g, tune, plan, false);
  return EHIP_OK;
}

}  // namespace ehip
