// LRU expert->slot tables on the GPU: acquire (one or two tables per launch),
// need mask, pack, prefill seeding and chunk planning.
//
// Rules follow ExpertTable (table.py:28-247) and the fused acquire kernel
// (acquire.py:25-141). Each table update runs in ONE workgroup: the need set,
// the victim keys and the miss ranks live in LDS, ranks come from wave
// ballots (mbcnt prefix counts) instead of a full sort, and only the first
// M (= number of misses) entries of the victim order are materialised.
#include "common.h"

namespace xp {
namespace {

constexpr int kThreads = 256;            // one workgroup per table
constexpr int kWaves = kThreads / 64;
constexpr int64_t kProtect = int64_t(1) << 40;  // table.py:16
constexpr int kSlotBits = 10;            // (key << 10) | slot keeps the sort stable for S <= 1024

struct TableDev {
  int64_t* slot_of;
  int64_t* expert_in;
  int64_t* last_used;
  int64_t* step;
  int64_t* hits;
  int64_t* misses;
  int E;
  int S;
};

TableDev to_dev(const xp_table* t) {
  return TableDev{t->slot_of, t->expert_in, t->last_used, t->step, t->hits, t->misses,
                  static_cast<int>(t->num_experts), static_cast<int>(t->num_slots)};
}

// LDS working set of one table update.
struct AcquireLds {
  uint8_t need[XP_MAX_EXPERTS];
  int16_t cur[XP_MAX_EXPERTS];    // slot_of before the update
  int16_t rank[XP_MAX_EXPERTS];   // ordinal of a miss (ascending expert id), -1 otherwise
  int16_t fin[XP_MAX_EXPERTS];    // slot_of after the update (for callers that chain updates)
  uint64_t key[XP_MAX_SLOTS];     // (last_used + used * 2^40) << 10 | slot
  int16_t occ[XP_MAX_SLOTS];      // expert_in before the update
  int16_t order[XP_MAX_SLOTS];    // order[r] = slot taken by the r-th miss
  int16_t miss_e[XP_MAX_SLOTS];   // miss_e[r] = the r-th missed expert
  int16_t ids[XP_MAX_SLOTS];      // the step's ids, -1 where not an expert
  int wave_a[kWaves];
  int wave_b[kWaves];
};

// Block-wide exclusive scan of two flags per thread (wave ballots + LDS
// wave totals). Returns prefix counts; totals via *ta / *tb. All threads of
// the block must call it.
__device__ __forceinline__ void block_scan2(bool fa, bool fb, int* pa, int* pb, int* ta, int* tb,
                                            int* wave_a, int* wave_b) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  unsigned long long ma = __ballot(fa), mb = __ballot(fb);
  if (lane == 0) {
    wave_a[wave] = __popcll(ma);
    wave_b[wave] = __popcll(mb);
  }
  __syncthreads();
  int ba = 0, bb = 0, sa = 0, sb = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    int ca = wave_a[w], cb = wave_b[w];
    if (w < wave) {
      ba += ca;
      bb += cb;
    }
    sa += ca;
    sb += cb;
  }
  *pa = ba + static_cast<int>(lane_prefix(ma));
  *pb = bb + static_cast<int>(lane_prefix(mb));
  *ta = sa;
  *tb = sb;
  __syncthreads();  // wave_a/wave_b may be reused by the next call
}

// One acquire on table `t` (table.py:75-128). `ids(k)` yields the k-th id of
// the step. Writes the outputs that are non-null. The table arrays may be in
// global memory or LDS (generic pointers). On return lds.fin holds slot_of
// after the update for every expert.
// slot_out: with slot_final, slot_of after the update for every expert (the
// torch version reads `current` through a view of slot_of, table.py:95-118);
// otherwise the fused kernel's value, the slot loaded before the update for
// experts that did not miss (acquire.py:309-341). Both agree on needed experts.
// The M smallest keys of key[0..S) in ascending order into order[], by one
// wave: M rounds of a wave-wide minimum (keys are distinct: the slot is in
// the low bits). Used when the misses are few.
__device__ __forceinline__ void smallest_keys_wave(const uint64_t* key, int S, int M, int16_t* order) {
  const int lane = threadIdx.x & 63;
  constexpr int kPer = XP_MAX_SLOTS / 64;
  uint64_t k[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int s = lane + 64 * i;
    k[i] = s < S ? key[s] : ~0ull;
  }
  for (int r = 0; r < M; ++r) {
    uint64_t m = k[0];
#pragma unroll
    for (int i = 1; i < kPer; ++i) m = k[i] < m ? k[i] : m;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const uint64_t o = static_cast<uint64_t>(__shfl_xor(static_cast<long long>(m), off, 64));
      m = o < m ? o : m;
    }
    if (lane == 0) order[r] = static_cast<int16_t>(m & ((1u << kSlotBits) - 1));
#pragma unroll
    for (int i = 0; i < kPer; ++i)
      if (k[i] == m) k[i] = ~0ull;
  }
}

// One acquire on table `t` (table.py:75-128). `ids(k)` yields the k-th id of
// the step. Writes the outputs that are non-null. The table arrays may be in
// global memory or LDS (generic pointers). On return lds.fin holds slot_of
// after the update for every expert.
// slot_out: with slot_final, slot_of after the update for every expert (the
// torch version reads `current` through a view of slot_of, table.py:95-118);
// otherwise the fused kernel's value, the slot loaded before the update for
// experts that did not miss (acquire.py:309-341). Both agree on needed experts.
template <typename Ids>
__device__ void acquire_block(Ids ids, int K, TableDev t, int64_t* map64, int32_t* map32,
                              int64_t* slot_out, int64_t* todo, bool count_refs, bool slot_final,
                              AcquireLds& lds) {
  const int tid = threadIdx.x;
  const int E = t.E, S = t.S;
  constexpr int kPerE = XP_MAX_EXPERTS / kThreads;
  constexpr int kPerS = XP_MAX_SLOTS / kThreads;

  // Every read of the table and of the ids is issued first, so the
  // latencies overlap (K <= S <= XP_MAX_SLOTS: kPerS ids per thread).
  int64_t cur_r[kPerE], occ_r[kPerS], lu_r[kPerS], id_r[kPerS];
#pragma unroll
  for (int i = 0; i < kPerE; ++i) {
    const int e = tid + kThreads * i;
    cur_r[i] = e < E ? t.slot_of[e] : -1;
  }
#pragma unroll
  for (int i = 0; i < kPerS; ++i) {
    const int s = tid + kThreads * i;
    occ_r[i] = s < S ? t.expert_in[s] : -1;
    lu_r[i] = s < S ? t.last_used[s] : 0;
  }
#pragma unroll
  for (int i = 0; i < kPerS; ++i) {
    const int k = tid + kThreads * i;
    id_r[i] = k < K ? ids(k) : -1;
  }
  const int64_t step = *t.step;
  // The counters too, so that their update at the end is not a global
  // round trip of its own.
  int64_t hits0 = 0, misses0 = 0;
  if (count_refs && tid == 0) {
    hits0 = *t.hits;
    misses0 = *t.misses;
  }

  for (int e = tid; e < E; e += kThreads) lds.need[e] = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kPerS; ++i) {
    const int k = tid + kThreads * i;
    if (k < K) {
      const int64_t id = id_r[i];
      const bool ok = id >= 0 && id < E;
      if (ok) lds.need[id] = 1;  // same value for duplicates
      lds.ids[k] = static_cast<int16_t>(ok ? id : -1);
    }
  }
  __syncthreads();

  // Victim keys: slots holding an expert needed this step are pushed to the
  // end (acquire.py:52-58, table.py:99-107). The slot number in the low bits
  // makes equal stamps order by slot, as the stable argsort does.
#pragma unroll
  for (int i = 0; i < kPerS; ++i) {
    const int s = tid + kThreads * i;
    if (s < S) {
      const int64_t occ = occ_r[i];
      const bool used = occ >= 0 && occ < E && lds.need[occ];
      const int64_t key = lu_r[i] + (used ? kProtect : 0);
      lds.key[s] = (static_cast<uint64_t>(key) << kSlotBits) | static_cast<uint64_t>(s);
      lds.occ[s] = static_cast<int16_t>(occ < 0 ? -1 : occ);
    }
  }

  // Hits and misses; the rank of a miss is its ordinal in ascending expert id.
  int miss_base = 0, hit_total = 0;
#pragma unroll
  for (int i = 0; i < kPerE; ++i) {
    const int e0 = kThreads * i;
    if (e0 >= E) break;  // uniform
    const int e = e0 + tid;
    const int64_t cur = cur_r[i];
    const bool n = e < E && lds.need[e];
    const bool miss = n && cur < 0, hit = n && cur >= 0;
    int pm, ph, tm, th;
    block_scan2(miss, hit, &pm, &ph, &tm, &th, lds.wave_a, lds.wave_b);
    if (e < E) {
      lds.cur[e] = static_cast<int16_t>(cur < 0 ? -1 : cur);
      lds.rank[e] = static_cast<int16_t>(miss ? miss_base + pm : -1);
    }
    if (miss) lds.miss_e[miss_base + pm] = static_cast<int16_t>(e);
    miss_base += tm;
    hit_total += th;
  }
  const int M = miss_base;  // <= K <= S (checked on the host)
  __syncthreads();

  // order[r] for r < M: the slot with the r-th smallest key. Either each
  // slot counts the keys below its own (S broadcast LDS reads per slot, S/256
  // slots per thread), or one wave takes M rounds of a wave-wide minimum
  // (about 1000 clocks a round): whichever is cheaper for this S and M.
  if (M > 0) {
    const int per = (S + kThreads - 1) / kThreads;
    if (M > 32 || S * per < 83 * M) {
      for (int s = tid; s < S; s += kThreads) {
        const uint64_t mine = lds.key[s];
        int c = 0, s2 = 0;
        for (; s2 + 8 <= S; s2 += 8) {  // eight reads in flight at a time
          uint64_t k8[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) k8[u] = lds.key[s2 + u];
#pragma unroll
          for (int u = 0; u < 8; ++u) c += k8[u] < mine ? 1 : 0;
        }
        for (; s2 < S; ++s2) c += lds.key[s2] < mine ? 1 : 0;
        if (c < M) lds.order[c] = static_cast<int16_t>(s);
      }
    } else if (tid < 64) {
      smallest_keys_wave(lds.key, S, M, lds.order);
    }
  }
  __syncthreads();

  // Evict the victims' occupants and move the misses in (table.py:112-116).
  // Victims are distinct and never hold a needed expert, so the writes of
  // different threads touch different elements.
  for (int r = tid; r < M; r += kThreads) {
    const int v = lds.order[r], e = lds.miss_e[r], old = lds.occ[v];
    if (old >= 0 && old < E) t.slot_of[old] = -1;
    t.slot_of[e] = v;
    t.expert_in[v] = e;
  }

  // Per-expert outputs and the last_used stamps (table.py:118-128).
  for (int e = tid; e < E; e += kThreads) {
    const int r = lds.rank[e];
    const int64_t slot = r >= 0 ? static_cast<int64_t>(lds.order[r]) : static_cast<int64_t>(lds.cur[e]);
    const bool n = lds.need[e];
    if (slot_out && !slot_final) slot_out[e] = slot;
    const int64_t mapped = n ? slot : -1;
    if (map64) map64[e] = mapped;
    if (map32) map32[e] = static_cast<int32_t>(mapped);
    if (n && slot >= 0 && slot < S) t.last_used[slot] = step;
    lds.fin[e] = static_cast<int16_t>(r >= 0 ? lds.order[r] : lds.cur[e]);
  }
  if (todo)
    for (int i = tid; i < K; i += kThreads) todo[i] = i < M ? static_cast<int64_t>(lds.miss_e[i]) : -1;
  __syncthreads();
  for (int r = tid; r < M; r += kThreads) {
    const int old = lds.occ[lds.order[r]];
    if (old >= 0 && old < E) lds.fin[old] = -1;
  }
  if (slot_out && slot_final) {
    __syncthreads();
    for (int e = tid; e < E; e += kThreads) slot_out[e] = lds.fin[e];
  }
  if (tid == 0) {
    *t.step = step + 1;
    if (count_refs) {
      *t.hits = hits0 + hit_total;
      *t.misses = misses0 + M;
    }
  }
  __syncthreads();
}

struct GlobalIds {
  const void* p;
  int eb;
  __device__ int64_t operator()(int k) const { return load_id(p, eb, k); }
};

__global__ void __launch_bounds__(kThreads) acquire_pair_kernel(GlobalIds ids, int K, TableDev a, TableDev b,
                                                                 int32_t* expert_map, int64_t* a_slot,
                                                                 int64_t* a_todo, int64_t* b_slot,
                                                                 int64_t* b_todo, int32_t* pair_slot) {
  __shared__ AcquireLds lds;
  if (blockIdx.x == 0) {
    acquire_block(ids, K, a, nullptr, expert_map, a_slot, a_todo, true, false, lds);
    // Each id's slot in table a, in step order: the expert FFN reads it in
    // one load instead of id then expert_map.
    if (pair_slot)
      for (int k = threadIdx.x; k < K; k += kThreads) {
        const int id = lds.ids[k];
        pair_slot[k] = id >= 0 ? static_cast<int32_t>(lds.fin[id]) : -1;
      }
  } else {
    acquire_block(ids, K, b, nullptr, nullptr, b_slot, b_todo, true, false, lds);
  }
}

__global__ void __launch_bounds__(kThreads) acquire_one_kernel(GlobalIds ids, int K, TableDev t, int64_t* map64,
                                                               int32_t* map32, int64_t* slot_out,
                                                               int64_t* todo) {
  __shared__ AcquireLds lds;
  acquire_block(ids, K, t, map64, map32, slot_out, todo, true, true, lds);
}

__global__ void __launch_bounds__(1024) need_mask_kernel(GlobalIds ids, int64_t n, int E, uint8_t* need) {
  __shared__ uint8_t s_need[XP_MAX_EXPERTS];
  for (int e = threadIdx.x; e < E; e += blockDim.x) s_need[e] = 0;
  __syncthreads();
  for (int64_t k = threadIdx.x; k < n; k += blockDim.x) {
    int64_t id = ids(static_cast<int>(k));
    if (id >= 0 && id < E) s_need[id] = 1;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) need[e] = s_need[e];
}

__global__ void __launch_bounds__(kThreads) pack_kernel(const uint8_t* mask, int E, int64_t* out) {
  __shared__ int wave_a[kWaves], wave_b[kWaves];
  int base = 0;
  for (int e0 = 0; e0 < E; e0 += kThreads) {
    const int e = e0 + threadIdx.x;
    const bool m = e < E && mask[e];
    int p, q, t, u;
    block_scan2(m, false, &p, &q, &t, &u, wave_a, wave_b);
    if (e < E) out[e] = -1;
    __syncthreads();
    if (m) out[base + p] = e;
    base += t;
  }
}

// ---- prefill seeding (table.py:140-171) ----

struct SeedLds {
  AcquireLds acq;
  int counts[XP_MAX_EXPERTS];
  int16_t top[XP_MAX_SLOTS];
  int16_t ids2[XP_MAX_SLOTS];
  int64_t slot_of[XP_MAX_EXPERTS + 1];
  int64_t expert_in[XP_MAX_SLOTS + 1];
  int64_t last_used[XP_MAX_SLOTS + 1];
  int64_t step, hits, misses;
};

struct LdsIds16 {
  const int16_t* p;
  __device__ int64_t operator()(int k) const { return p[k]; }
};

__global__ void __launch_bounds__(kThreads) seed_kernel(TableDev ram, TableDev vram, GlobalIds ids, int64_t n,
                                                        const uint8_t* need) {
  extern __shared__ unsigned char smem_raw[];
  SeedLds& lds = *reinterpret_cast<SeedLds*>(smem_raw);
  const int tid = threadIdx.x;
  const int E = ram.E, R = ram.S, S = vram.S;

  // Work on an LDS copy of the RAM table so both acquires see each other's
  // writes without a global round trip; copy back at the end.
  for (int e = tid; e < E; e += kThreads) lds.slot_of[e] = ram.slot_of[e];
  for (int s = tid; s < R; s += kThreads) {
    lds.expert_in[s] = ram.expert_in[s];
    lds.last_used[s] = ram.last_used[s];
  }
  for (int e = tid; e < E; e += kThreads) lds.counts[e] = 0;
  if (tid == 0) lds.step = *ram.step;
  __syncthreads();
  for (int64_t k = tid; k < n; k += kThreads) {
    int64_t id = ids(static_cast<int>(k));
    if (id >= 0 && id < E) atomicAdd(&lds.counts[id], 1);
  }
  __syncthreads();

  // The max(R - S, 1) most referenced experts; ties go to the lower expert id
  // (torch.topk leaves the tie order unspecified, table.py:161).
  const int ntop = R - S > 1 ? R - S : 1;
  for (int e = tid; e < E; e += kThreads) {
    const int c = lds.counts[e];
    int r = 0;
    for (int e2 = 0; e2 < E; ++e2) {
      const int c2 = lds.counts[e2];
      r += (c2 > c || (c2 == c && e2 < e)) ? 1 : 0;
    }
    if (r < ntop) lds.top[r] = static_cast<int16_t>(e);
  }
  __syncthreads();
  // Unreferenced picks become the most referenced expert (table.py:162-164).
  const int16_t top0 = lds.top[0];
  for (int i = tid; i < ntop; i += kThreads)
    if (lds.counts[lds.top[i]] <= 0) lds.top[i] = top0;
  __syncthreads();

  TableDev t{lds.slot_of, lds.expert_in, lds.last_used, &lds.step, &lds.hits, &lds.misses, E, R};
  if (R > S) acquire_block(LdsIds16{lds.top}, ntop, t, nullptr, nullptr, nullptr, nullptr, false, true, lds.acq);

  // Then the VRAM tier's experts that have a row to read: in RAM after the
  // first acquire, or referenced this step (table.py:167-169).
  for (int s = tid; s < S; s += kThreads) {
    const int64_t v = vram.expert_in[s];
    const bool ok = v >= 0 && v < E && (lds.slot_of[v] >= 0 || need[v]);
    lds.ids2[s] = ok ? static_cast<int16_t>(v) : top0;
  }
  __syncthreads();
  acquire_block(LdsIds16{lds.ids2}, S, t, nullptr, nullptr, nullptr, nullptr, false, true, lds.acq);

  for (int e = tid; e < E; e += kThreads) ram.slot_of[e] = lds.slot_of[e];
  for (int s = tid; s < R; s += kThreads) {
    ram.expert_in[s] = lds.expert_in[s];
    ram.last_used[s] = lds.last_used[s];
  }
  if (tid == 0) *ram.step = lds.step;
}

// ---- chunk planning (table.py:173-247) ----

__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {
  int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}
__device__ __forceinline__ int64_t floor_mod(int64_t a, int64_t b) { return a - floor_div(a, b) * b; }

struct PlanLds {
  int a[XP_MAX_EXPERTS];  // inclusive cumsum of `first`
  int b[XP_MAX_EXPERTS];  // inclusive cumsum of `ssd`
  uint8_t old_ok[XP_MAX_EXPERTS];
  uint8_t ssd[XP_MAX_EXPERTS];
  uint8_t first[XP_MAX_EXPERTS];
  int wave_a[kWaves], wave_b[kWaves];
};

__global__ void __launch_bounds__(kThreads) plan_kernel(const int64_t* slot_of, int E, const int64_t* before,
                                                        const uint8_t* need, const int64_t* cached_row, int64_t W,
                                                        int64_t ram_base, int64_t working_base, int64_t* dst_row,
                                                        int64_t* src_row, int64_t* maps, int64_t* todo,
                                                        int64_t* ssd_out, int64_t* late) {
  __shared__ PlanLds lds;
  const int tid = threadIdx.x;
  const int64_t N = (E + W - 1) / W + 1;
  int ra = 0, rb = 0;
  for (int e0 = 0; e0 < E; e0 += kThreads) {
    const int e = e0 + tid;
    bool first = false, ssd = false, ok = false;
    if (e < E) {
      const int64_t bf = before[e], af = slot_of[e];
      ok = bf >= 0 && (af < 0 || af == bf);
      ssd = !ok && (need[e] || bf >= 0);
      first = need[e] && !ssd;
    }
    int pa, pb, ta, tb;
    block_scan2(first, ssd, &pa, &pb, &ta, &tb, lds.wave_a, lds.wave_b);
    if (e < E) {
      lds.a[e] = ra + pa + (first ? 1 : 0);
      lds.b[e] = rb + pb + (ssd ? 1 : 0);
      lds.old_ok[e] = ok;
      lds.ssd[e] = ssd;
      lds.first[e] = first;
    }
    ra += ta;
    rb += tb;
  }
  __syncthreads();
  const int64_t boundary = (static_cast<int64_t>(ra) + W - 1) / W * W;
  for (int64_t i = tid; i < N * W; i += kThreads) todo[i] = ssd_out[i] = late[i] = -1;
  __syncthreads();
  for (int e = tid; e < E; e += kThreads) {
    const int64_t pos = lds.first[e] ? lds.a[e] - 1 : boundary + lds.b[e] - 1;
    const int64_t drow = floor_mod(pos, W);
    const int64_t shared = working_base + floor_mod(floor_div(pos, W), 2) * W + drow;
    const int64_t bf = before[e], af = slot_of[e];
    dst_row[e] = drow;
    src_row[e] = lds.old_ok[e] ? bf + ram_base : (af >= 0 ? af + ram_base : shared);
    const bool nd = need[e];
    const int64_t chunk = nd ? floor_div(pos, W) : -1;
    for (int64_t k = 0; k < N; ++k) maps[k * E + e] = chunk == k ? drow : -1;
    const bool s = lds.ssd[e];
    if (nd && (!s || cached_row[e] >= 0)) todo[pos] = e;
    if (s) ssd_out[pos] = e;
    if (nd && s && cached_row[e] < 0) late[pos] = e;
  }
}

}  // namespace
}  // namespace xp

using namespace xp;

static int check_table(const xp_table* t, const char* what) {
  XP_REQUIRE(t != nullptr && t->slot_of && t->expert_in && t->last_used && t->step && t->hits && t->misses,
             "%s: table pointers must be non-null", what);
  XP_REQUIRE(t->num_experts >= 1 && t->num_experts <= XP_MAX_EXPERTS, "%s: %lld experts (1..%d supported)", what,
             (long long)t->num_experts, XP_MAX_EXPERTS);
  XP_REQUIRE(t->num_slots >= 1 && t->num_slots <= XP_MAX_SLOTS, "%s: %lld slots (1..%d supported)", what,
             (long long)t->num_slots, XP_MAX_SLOTS);
  return XP_OK;
}

static int check_ids(const void* topk, int eb, int64_t n, const char* what) {
  XP_REQUIRE(eb == 4 || eb == 8, "%s: topk element size %d (4 or 8)", what, eb);
  XP_REQUIRE(n >= 0 && n <= (int64_t(1) << 30), "%s: %lld ids", what, (long long)n);
  XP_REQUIRE(n == 0 || topk != nullptr, "%s: null topk", what);
  return XP_OK;
}

extern "C" {

int xp_acquire_pair(const void* topk, int topk_elem_bytes, int64_t K, const xp_table* vram, const xp_table* ram,
                    int32_t* expert_map, int64_t* vram_slot, int64_t* vram_todo, int64_t* ram_slot,
                    int64_t* ram_todo, int32_t* pair_slot, void* stream) {
  int rc;
  if ((rc = check_ids(topk, topk_elem_bytes, K, "xp_acquire_pair")) ||
      (rc = check_table(vram, "xp_acquire_pair(vram)")) || (rc = check_table(ram, "xp_acquire_pair(ram)")))
    return rc;
  XP_REQUIRE(vram->num_experts == ram->num_experts, "xp_acquire_pair: tables have %lld and %lld experts",
             (long long)vram->num_experts, (long long)ram->num_experts);
  XP_REQUIRE(K <= vram->num_slots && K <= ram->num_slots,
             "xp_acquire_pair: %lld ids exceed the slots (%lld, %lld)", (long long)K, (long long)vram->num_slots,
             (long long)ram->num_slots);
  XP_REQUIRE(expert_map && vram_slot && vram_todo && ram_slot && ram_todo, "xp_acquire_pair: null output");
  hipLaunchKernelGGL(acquire_pair_kernel, dim3(2), dim3(kThreads), 0, as_stream(stream),
                     GlobalIds{topk, topk_elem_bytes}, static_cast<int>(K), to_dev(vram), to_dev(ram), expert_map,
                     vram_slot, vram_todo, ram_slot, ram_todo, pair_slot);
  return check_launch("acquire_pair_kernel");
}

int xp_table_acquire(const void* topk, int topk_elem_bytes, int64_t K, const xp_table* t, int64_t* expert_map_i64,
                     int32_t* expert_map_i32, int64_t* slot_out, int64_t* todo, void* stream) {
  int rc;
  if ((rc = check_ids(topk, topk_elem_bytes, K, "xp_table_acquire")) || (rc = check_table(t, "xp_table_acquire")))
    return rc;
  XP_REQUIRE(K <= t->num_slots, "xp_table_acquire: %lld ids exceed %lld slots", (long long)K,
             (long long)t->num_slots);
  hipLaunchKernelGGL(acquire_one_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream),
                     GlobalIds{topk, topk_elem_bytes}, static_cast<int>(K), to_dev(t), expert_map_i64,
                     expert_map_i32, slot_out, todo);
  return check_launch("acquire_one_kernel");
}

int xp_need_mask(const void* topk, int topk_elem_bytes, int64_t n, int64_t num_experts, uint8_t* need,
                 void* stream) {
  int rc;
  if ((rc = check_ids(topk, topk_elem_bytes, n, "xp_need_mask"))) return rc;
  XP_REQUIRE(num_experts >= 1 && num_experts <= XP_MAX_EXPERTS && need, "xp_need_mask: bad arguments");
  hipLaunchKernelGGL(need_mask_kernel, dim3(1), dim3(1024), 0, as_stream(stream), GlobalIds{topk, topk_elem_bytes},
                     n, static_cast<int>(num_experts), need);
  return check_launch("need_mask_kernel");
}

int xp_pack(const uint8_t* mask, int64_t num_experts, int64_t* out, void* stream) {
  XP_REQUIRE(mask && out && num_experts >= 1 && num_experts <= XP_MAX_EXPERTS, "xp_pack: bad arguments");
  hipLaunchKernelGGL(pack_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream), mask,
                     static_cast<int>(num_experts), out);
  return check_launch("pack_kernel");
}

int xp_table_seed(const xp_table* ram, const xp_table* vram, const void* topk, int topk_elem_bytes, int64_t n,
                  const uint8_t* need, void* stream) {
  int rc;
  if ((rc = check_ids(topk, topk_elem_bytes, n, "xp_table_seed")) || (rc = check_table(ram, "xp_table_seed(ram)")) ||
      (rc = check_table(vram, "xp_table_seed(vram)")))
    return rc;
  XP_REQUIRE(ram->num_experts == vram->num_experts, "xp_table_seed: expert counts differ");
  XP_REQUIRE(vram->num_slots <= ram->num_slots, "xp_table_seed: VRAM slots (%lld) exceed RAM slots (%lld)",
             (long long)vram->num_slots, (long long)ram->num_slots);
  XP_REQUIRE(ram->num_slots <= ram->num_experts, "xp_table_seed: %lld RAM slots exceed %lld experts",
             (long long)ram->num_slots, (long long)ram->num_experts);
  XP_REQUIRE(need != nullptr, "xp_table_seed: null need mask");
  const size_t smem = sizeof(SeedLds);
  XP_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(seed_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                             static_cast<int>(smem)));
  hipLaunchKernelGGL(seed_kernel, dim3(1), dim3(kThreads), smem, as_stream(stream), to_dev(ram), to_dev(vram),
                     GlobalIds{topk, topk_elem_bytes}, n, need);
  return check_launch("seed_kernel");
}

int xp_plan_chunks(const xp_table* ram, const int64_t* before, const uint8_t* need, const int64_t* cached_row,
                   int64_t W, int64_t ram_base, int64_t working_base, int64_t* dst_row, int64_t* src_row,
                   int64_t* maps, int64_t* todo, int64_t* ssd, int64_t* late, void* stream) {
  int rc;
  if ((rc = check_table(ram, "xp_plan_chunks"))) return rc;
  XP_REQUIRE(W >= 1, "xp_plan_chunks: W=%lld", (long long)W);
  XP_REQUIRE(before && need && cached_row && dst_row && src_row && maps && todo && ssd && late,
             "xp_plan_chunks: null argument");
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream), ram->slot_of,
                     static_cast<int>(ram->num_experts), before, need, cached_row, W, ram_base, working_base, dst_row,
                     src_row, maps, todo, ssd, late);
  return check_launch("plan_kernel");
}

}  // extern "C"
