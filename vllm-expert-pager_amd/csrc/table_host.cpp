// ExpertTable rules on host memory, for tables kept in CPU tensors.
//
// The reference's ExpertTable is written in device-agnostic torch ops, so its
// tables also run on CPU tensors, where its own tests drive them
// (table.py:1-9). These are the same rules as the single-workgroup kernels
// of table.hip, written as sequential loops over host arrays; they give the
// same table state and outputs element for element (tests compare both with
// the oracle). A table on a GPU never takes this path.
#include <algorithm>
#include <cstdint>
#include <vector>

#include "../../include/xp.h"

namespace xp {
int fail(int code, const char* fmt, ...);
}

namespace {

constexpr int64_t kProtect = int64_t(1) << 40;  // table.py:16

#define XPH_REQUIRE(cond, ...) \
  do {                         \
    if (!(cond)) return xp::fail(XP_E_ARG, __VA_ARGS__); \
  } while (0)

int64_t id_at(const void* p, int eb, int64_t k) {
  return eb == 4 ? static_cast<const int32_t*>(p)[k] : static_cast<const int64_t*>(p)[k];
}

int check_table(const xp_table* t, const char* what) {
  XPH_REQUIRE(t != nullptr && t->slot_of && t->expert_in && t->last_used && t->step && t->hits && t->misses,
              "%s: table pointers must be non-null", what);
  XPH_REQUIRE(t->num_experts >= 1 && t->num_experts <= XP_MAX_EXPERTS, "%s: %lld experts (1..%d supported)", what,
              (long long)t->num_experts, XP_MAX_EXPERTS);
  XPH_REQUIRE(t->num_slots >= 1 && t->num_slots <= XP_MAX_SLOTS, "%s: %lld slots (1..%d supported)", what,
              (long long)t->num_slots, XP_MAX_SLOTS);
  return XP_OK;
}

int check_ids(const void* topk, int eb, int64_t n, const char* what) {
  XPH_REQUIRE(eb == 4 || eb == 8, "%s: topk element size %d (4 or 8)", what, eb);
  XPH_REQUIRE(n >= 0 && n <= (int64_t(1) << 30), "%s: %lld ids", what, (long long)n);
  XPH_REQUIRE(n == 0 || topk != nullptr, "%s: null topk", what);
  return XP_OK;
}

// One acquire (table.py:75-128): the needed experts that miss take, in
// ascending expert id, the slots with the smallest (last_used + protect if it
// holds a needed expert, slot) keys. slot_out gets slot_of after the update.
// count_refs adds the step's hits and misses to the counters.
void acquire(const std::vector<int64_t>& ids, const xp_table& t, int64_t* map64, int32_t* map32, int64_t* slot_out,
             int64_t* todo, bool count_refs) {
  const int64_t E = t.num_experts, S = t.num_slots, K = static_cast<int64_t>(ids.size());
  std::vector<uint8_t> need(static_cast<size_t>(E), 0);
  for (int64_t id : ids)
    if (id >= 0 && id < E) need[static_cast<size_t>(id)] = 1;
  const std::vector<int64_t> cur(t.slot_of, t.slot_of + E);
  std::vector<std::pair<int64_t, int64_t>> key(static_cast<size_t>(S));  // (key, slot)
  for (int64_t s = 0; s < S; ++s) {
    const int64_t occ = t.expert_in[s];
    const bool used = occ >= 0 && occ < E && need[static_cast<size_t>(occ)];
    key[static_cast<size_t>(s)] = {t.last_used[s] + (used ? kProtect : 0), s};
  }
  std::vector<int64_t> miss_e, rank(static_cast<size_t>(E), -1);
  int64_t hits = 0;
  for (int64_t e = 0; e < E; ++e) {
    if (!need[static_cast<size_t>(e)]) continue;
    if (cur[static_cast<size_t>(e)] >= 0) {
      ++hits;
    } else {
      rank[static_cast<size_t>(e)] = static_cast<int64_t>(miss_e.size());
      miss_e.push_back(e);
    }
  }
  const int64_t M = static_cast<int64_t>(miss_e.size());  // <= K <= S
  std::stable_sort(key.begin(), key.end());
  std::vector<int64_t> victim(static_cast<size_t>(M)), evicted(static_cast<size_t>(M));
  for (int64_t r = 0; r < M; ++r) {
    victim[static_cast<size_t>(r)] = key[static_cast<size_t>(r)].second;
    evicted[static_cast<size_t>(r)] = t.expert_in[victim[static_cast<size_t>(r)]];
  }
  for (int64_t r = 0; r < M; ++r) {  // victims never hold a needed expert
    const int64_t old = evicted[static_cast<size_t>(r)];
    if (old >= 0 && old < E) t.slot_of[old] = -1;
  }
  for (int64_t r = 0; r < M; ++r) {
    const int64_t v = victim[static_cast<size_t>(r)], e = miss_e[static_cast<size_t>(r)];
    t.slot_of[e] = v;
    t.expert_in[v] = e;
  }
  const int64_t step = *t.step;
  for (int64_t e = 0; e < E; ++e) {
    const int64_t r = rank[static_cast<size_t>(e)];
    const int64_t slot = r >= 0 ? victim[static_cast<size_t>(r)] : cur[static_cast<size_t>(e)];
    const bool n = need[static_cast<size_t>(e)];
    const int64_t mapped = n ? slot : -1;
    if (map64) map64[e] = mapped;
    if (map32) map32[e] = static_cast<int32_t>(mapped);
    if (n && slot >= 0 && slot < S) t.last_used[slot] = step;
  }
  if (slot_out)
    for (int64_t e = 0; e < E; ++e) slot_out[e] = t.slot_of[e];
  if (todo)
    for (int64_t i = 0; i < K; ++i) todo[i] = i < M ? miss_e[static_cast<size_t>(i)] : -1;
  *t.step = step + 1;
  if (count_refs) {
    *t.hits += hits;
    *t.misses += M;
  }
}

std::vector<int64_t> read_ids(const void* topk, int eb, int64_t n) {
  std::vector<int64_t> ids(static_cast<size_t>(n));
  for (int64_t k = 0; k < n; ++k) ids[static_cast<size_t>(k)] = id_at(topk, eb, k);
  return ids;
}

int64_t floor_div(int64_t a, int64_t b) {
  const int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}
int64_t floor_mod(int64_t a, int64_t b) { return a - floor_div(a, b) * b; }

}  // namespace

extern "C" {

int xp_table_acquire_host(const void* topk, int topk_elem_bytes, int64_t K, const xp_table* t,
                          int64_t* expert_map_i64, int32_t* expert_map_i32, int64_t* slot_out, int64_t* todo) {
  int rc;
  if ((rc = check_ids(topk, topk_elem_bytes, K, "xp_table_acquire_host")) ||
      (rc = check_table(t, "xp_table_acquire_host")))
    return rc;
  XPH_REQUIRE(K <= t->num_slots, "xp_table_acquire_host: %lld ids exceed %lld slots", (long long)K,
              (long long)t->num_slots);
  acquire(read_ids(topk, topk_elem_bytes, K), *t, expert_map_i64, expert_map_i32, slot_out, todo, true);
  return XP_OK;
}

int xp_need_mask_host(const void* topk, int topk_elem_bytes, int64_t n, int64_t num_experts, uint8_t* need) {
  int rc;
  if ((rc = check_ids(topk, topk_elem_bytes, n, "xp_need_mask_host"))) return rc;
  XPH_REQUIRE(num_experts >= 1 && num_experts <= XP_MAX_EXPERTS && need, "xp_need_mask_host: bad arguments");
  std::fill(need, need + num_experts, uint8_t{0});
  for (int64_t k = 0; k < n; ++k) {
    const int64_t id = id_at(topk, topk_elem_bytes, k);
    if (id >= 0 && id < num_experts) need[id] = 1;
  }
  return XP_OK;
}

int xp_pack_host(const uint8_t* mask, int64_t num_experts, int64_t* out) {
  XPH_REQUIRE(mask && out && num_experts >= 1 && num_experts <= XP_MAX_EXPERTS, "xp_pack_host: bad arguments");
  int64_t r = 0;
  std::fill(out, out + num_experts, int64_t{-1});
  for (int64_t e = 0; e < num_experts; ++e)
    if (mask[e]) out[r++] = e;
  return XP_OK;
}

int xp_table_seed_host(const xp_table* ram, const xp_table* vram, const void* topk, int topk_elem_bytes, int64_t n,
                       const uint8_t* need) {
  int rc;
  if ((rc = check_ids(topk, topk_elem_bytes, n, "xp_table_seed_host")) ||
      (rc = check_table(ram, "xp_table_seed_host(ram)")) || (rc = check_table(vram, "xp_table_seed_host(vram)")))
    return rc;
  XPH_REQUIRE(ram->num_experts == vram->num_experts, "xp_table_seed_host: expert counts differ");
  XPH_REQUIRE(vram->num_slots <= ram->num_slots, "xp_table_seed_host: VRAM slots (%lld) exceed RAM slots (%lld)",
              (long long)vram->num_slots, (long long)ram->num_slots);
  XPH_REQUIRE(ram->num_slots <= ram->num_experts, "xp_table_seed_host: %lld RAM slots exceed %lld experts",
              (long long)ram->num_slots, (long long)ram->num_experts);
  XPH_REQUIRE(need != nullptr, "xp_table_seed_host: null need mask");
  const int64_t E = ram->num_experts, R = ram->num_slots, S = vram->num_slots;
  std::vector<int64_t> counts(static_cast<size_t>(E), 0);
  for (int64_t k = 0; k < n; ++k) {
    const int64_t id = id_at(topk, topk_elem_bytes, k);
    if (id >= 0 && id < E) ++counts[static_cast<size_t>(id)];
  }
  // The max(R - S, 1) most referenced experts, ties to the lower expert id
  // (torch.topk leaves the tie order unspecified, table.py:161); picks never
  // referenced become the most referenced one (table.py:162-164).
  const int64_t ntop = R - S > 1 ? R - S : 1;
  std::vector<int64_t> order(static_cast<size_t>(E));
  for (int64_t e = 0; e < E; ++e) order[static_cast<size_t>(e)] = e;
  std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) {
    return counts[static_cast<size_t>(a)] > counts[static_cast<size_t>(b)];
  });
  std::vector<int64_t> top(order.begin(), order.begin() + ntop);
  for (int64_t& e : top)
    if (counts[static_cast<size_t>(e)] <= 0) e = order[0];
  // The step's counters are not touched by seeding.
  if (R > S) acquire(top, *ram, nullptr, nullptr, nullptr, nullptr, false);
  // Then the VRAM tier's experts that have a row to read: in RAM after the
  // first acquire, or referenced this step (table.py:167-169).
  std::vector<int64_t> ids2(static_cast<size_t>(S));
  for (int64_t s = 0; s < S; ++s) {
    const int64_t v = vram->expert_in[s];
    const bool ok = v >= 0 && v < E && (ram->slot_of[v] >= 0 || need[v]);
    ids2[static_cast<size_t>(s)] = ok ? v : order[0];
  }
  acquire(ids2, *ram, nullptr, nullptr, nullptr, nullptr, false);
  return XP_OK;
}

int xp_plan_chunks_host(const xp_table* ram, const int64_t* before, const uint8_t* need, const int64_t* cached_row,
                        int64_t W, int64_t ram_base, int64_t working_base, int64_t* dst_row, int64_t* src_row,
                        int64_t* maps, int64_t* todo, int64_t* ssd, int64_t* late) {
  int rc;
  if ((rc = check_table(ram, "xp_plan_chunks_host"))) return rc;
  XPH_REQUIRE(W >= 1, "xp_plan_chunks_host: W=%lld", (long long)W);
  XPH_REQUIRE(before && need && cached_row && dst_row && src_row && maps && todo && ssd && late,
              "xp_plan_chunks_host: null argument");
  const int64_t E = ram->num_experts, N = (E + W - 1) / W + 1;
  std::vector<int64_t> a(static_cast<size_t>(E)), b(static_cast<size_t>(E));
  std::vector<uint8_t> old_ok(static_cast<size_t>(E)), is_ssd(static_cast<size_t>(E)), first(static_cast<size_t>(E));
  int64_t ra = 0, rb = 0;
  for (int64_t e = 0; e < E; ++e) {
    const int64_t bf = before[e], af = ram->slot_of[e];
    const bool ok = bf >= 0 && (af < 0 || af == bf);
    const bool s = !ok && (need[e] || bf >= 0);
    const bool f = need[e] && !s;
    ra += f;
    rb += s;
    a[static_cast<size_t>(e)] = ra;
    b[static_cast<size_t>(e)] = rb;
    old_ok[static_cast<size_t>(e)] = ok;
    is_ssd[static_cast<size_t>(e)] = s;
    first[static_cast<size_t>(e)] = f;
  }
  const int64_t boundary = (ra + W - 1) / W * W;
  std::fill(todo, todo + N * W, int64_t{-1});
  std::fill(ssd, ssd + N * W, int64_t{-1});
  std::fill(late, late + N * W, int64_t{-1});
  for (int64_t e = 0; e < E; ++e) {
    const size_t i = static_cast<size_t>(e);
    const int64_t pos = first[i] ? a[i] - 1 : boundary + b[i] - 1;
    const int64_t drow = floor_mod(pos, W);
    const int64_t shared = working_base + floor_mod(floor_div(pos, W), 2) * W + drow;
    const int64_t bf = before[e], af = ram->slot_of[e];
    dst_row[e] = drow;
    src_row[e] = old_ok[i] ? bf + ram_base : (af >= 0 ? af + ram_base : shared);
    const bool nd = need[e];
    const int64_t chunk = nd ? floor_div(pos, W) : -1;
    for (int64_t k = 0; k < N; ++k) maps[k * E + e] = chunk == k ? drow : -1;
    const bool s = is_ssd[i];
    if (nd && (!s || cached_row[e] >= 0)) todo[pos] = e;
    if (s) ssd[pos] = e;
    if (nd && s && cached_row[e] < 0) late[pos] = e;
  }
  return XP_OK;
}

}  // extern "C"
