// Slot gather (RAM tier / cache slab -> slab or staging) and the device half
// of the host request ring.
//
// Semantics follow gather_rows / _gather_rows_kernel (gather.py:51-194, 328-393)
// and the fetch kernels (gather.py:197-311, 396-439). The copy is done by a
// fixed number of persistent workgroups that walk the (row, 16 KiB chunk)
// sequence round-robin, each thread keeping four 16-byte loads in flight: the
// request depth over the host link is blocks x 16 KiB, tunable with
// xp_gather_set_blocks. The fetch half publishes a request into pinned
// coherent memory with a system-scope release store and polls `done` with a
// wall-clock deadline (s_sleep between polls) instead of a spin count.
#include "common.h"

namespace xp {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;                                  // 16-byte loads in flight per thread
constexpr int64_t kChunk = int64_t(kThreads) * kUnroll * 16;  // 16 KiB per workgroup step

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct NameDev {
  const uint8_t* src;
  int64_t src_pitch;
  int64_t src_rows;
  const uint8_t* cache;
  int64_t cache_rows;
  uint8_t* dst;
  int64_t dst_rows;
  int64_t row_bytes;
  uint8_t* stg;
  int64_t stg_rows;
  const uint8_t* scale;
  uint8_t* scale_dst;
  int64_t scale_bytes;
};

struct RingDev {
  int64_t* req;
  int64_t* done;
  int64_t* seq;
  int64_t block;
  int64_t ring;
};

struct GatherArgs {
  const int64_t* todo;
  int K;
  int E;
  const int64_t* dst_row;
  const int64_t* cache_row;
  const int64_t* src_row;
  int64_t base;
  NameDev names[2];
  int num_names;
  const int64_t* ssd;  // experts skipped by the copy (published by the fetch block)
  int fetch;           // 1: the last workgroup publishes ssd and waits
  int64_t layer;
  RingDev ring;
  int64_t retry_ticks;
  int64_t giveup;
};

// Copy `n` bytes (multiple of 4) from src to dst with 16-byte accesses where
// both are 16-byte aligned, by all threads of the workgroup.
__device__ __forceinline__ void copy_bytes(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, int64_t n) {
  const int tid = threadIdx.x;
  const bool vec = ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) == 0;
  int64_t done_bytes = 0;
  if (vec) {
    const int64_t nv = n >> 4;
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
    u32x4* d = reinterpret_cast<u32x4*>(dst);
    int64_t i = tid;
    for (; i + (kUnroll - 1) * kThreads < nv; i += kUnroll * kThreads) {
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = __builtin_nontemporal_load(s + i + u * kThreads);
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) d[i + u * kThreads] = v[u];
    }
    for (; i < nv; i += kThreads) d[i] = __builtin_nontemporal_load(s + i);
    done_bytes = nv << 4;
  }
  const uint32_t* s4 = reinterpret_cast<const uint32_t*>(src + done_bytes);
  uint32_t* d4 = reinterpret_cast<uint32_t*>(dst + done_bytes);
  for (int64_t i = tid; i < ((n - done_bytes) >> 2); i += kThreads) d4[i] = s4[i];
}

// True if some entry of list[0..K) is >= 0 (all threads of the block call it).
__device__ bool block_any_valid(const int64_t* list, int K) {
  __shared__ int s_any;
  if (threadIdx.x == 0) s_any = 0;
  __syncthreads();
  for (int k = threadIdx.x; k < K; k += blockDim.x)
    if (list[k] >= 0) s_any = 1;
  __syncthreads();
  const int any = s_any;
  __syncthreads();
  return any != 0;
}

__device__ __forceinline__ int64_t sys_load(const int64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void sys_store(int64_t* p, int64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Publish the experts of todo[0..K) (gather.py:197-234). Only the GPU writes
// req, so the counters are advanced with plain system-scope load/store pairs
// (no host-link read-modify-write atomics are needed).
__device__ void fetch_publish(const int64_t* todo, int K, int E, const int64_t* row, int64_t base, int64_t layer,
                              const RingDev& r, int64_t* ticket) {
  __shared__ int64_t s_seq;
  if (!block_any_valid(todo, K)) return;
  if (threadIdx.x == 0) {
    const int64_t seq = *r.seq + 1;
    *r.seq = seq;
    *ticket = seq;
    s_seq = seq;
  }
  __syncthreads();
  const int64_t seq = s_seq;
  int64_t* slot = r.req + 2 + (seq % r.ring) * (2 + 2 * r.block);
  // Every entry of the slot is written, so nothing of an earlier request is
  // left behind (gather.py:224-227).
  for (int64_t i = threadIdx.x; i < r.block; i += blockDim.x) {
    const int64_t e = i < K ? todo[i] : -1;
    const int64_t rowv = (e >= 0 && e < E) ? row[e] + base : -1;
    slot[2 + i] = e;
    slot[2 + r.block + i] = rowv;
  }
  if (threadIdx.x == 0) slot[1] = layer;
  __threadfence_system();
  __syncthreads();
  if (threadIdx.x == 0) sys_store(slot, seq);
}

// Wait for done >= ticket (gather.py:237-277): poll with s_sleep; every
// retry_ticks of the constant clock re-publish the slot and count it in
// req[0]; after `giveup` re-publishes stop and count it in req[1].
__device__ void fetch_wait(const int64_t* todo, int K, const RingDev& r, const int64_t* ticket, int64_t retry_ticks,
                           int64_t giveup) {
  if (!block_any_valid(todo, K)) return;
  if (threadIdx.x != 0) return;
  const int64_t seq = *ticket;
  int64_t* slot = r.req + 2 + (seq % r.ring) * (2 + 2 * r.block);
  int64_t d = sys_load(r.done);
  int64_t t0 = static_cast<int64_t>(wall_clock64());
  int64_t tries = 0;
  while (d < seq && tries < giveup) {
    __builtin_amdgcn_s_sleep(8);
    const int64_t now = static_cast<int64_t>(wall_clock64());
    if (now - t0 >= retry_ticks) {
      t0 = now;
      ++tries;
      sys_store(slot, seq);
      sys_store(r.req, sys_load(r.req) + 1);
    }
    d = sys_load(r.done);
  }
  if (d < seq) sys_store(r.req + 1, sys_load(r.req + 1) + 1);
}

__global__ void __launch_bounds__(kThreads) gather_kernel(GatherArgs a) {
  const int nblocks = a.fetch ? static_cast<int>(gridDim.x) - 1 : static_cast<int>(gridDim.x);
  const int b = blockIdx.x;
  if (a.fetch && b == nblocks) {
    fetch_publish(a.ssd, a.K, a.E, a.src_row, a.base, a.layer, a.ring, a.ring.seq);
    fetch_wait(a.ssd, a.K, a.ring, a.ring.seq, a.retry_ticks, a.giveup);
    return;
  }
  int64_t item = 0;  // running chunk index over the rows, for the round-robin
  for (int j = 0; j < a.K; ++j) {
    const int64_t e = a.todo[j];
    bool active = e >= 0 && e < a.E;
    if (active && a.fetch)
      for (int k = 0; k < a.K; ++k) active = active && a.ssd[k] != e;
    if (!active) continue;
    const int64_t drow = a.dst_row[e];
    const int64_t crow = a.cache_row[e];
    const int64_t srow = a.src_row[e] + a.base;
    for (int n = 0; n < a.num_names; ++n) {
      const NameDev& nm = a.names[n];
      const uint8_t* src;
      uint8_t* dst;
      int64_t len;
      // An expert whose destination row is outside [0, dst_rows) is not
      // copied at all (rows, staging or scales).
      const bool in_dst = drow >= 0 && drow < nm.dst_rows;
      bool ok;
      if (crow >= 0) {
        ok = crow < nm.cache_rows && in_dst;
        src = nm.cache + crow * nm.row_bytes;
        dst = nm.dst + drow * nm.row_bytes;
        len = nm.row_bytes;
      } else if (nm.stg) {
        ok = srow >= 0 && srow < nm.src_rows && j < nm.stg_rows && in_dst;
        src = nm.src + srow * nm.src_pitch;
        dst = nm.stg + int64_t(j) * nm.src_pitch;
        len = nm.src_pitch;
      } else {
        ok = srow >= 0 && srow < nm.src_rows && in_dst;
        src = nm.src + srow * nm.src_pitch;
        dst = nm.dst + drow * nm.row_bytes;
        len = nm.src_pitch;
      }
      const int64_t nchunks = (len + kChunk - 1) / kChunk;
      if (ok) {
        for (int64_t c = (b - item % nblocks + nblocks) % nblocks; c < nchunks; c += nblocks) {
          const int64_t off = c * kChunk;
          const int64_t cnt = len - off < kChunk ? len - off : kChunk;
          copy_bytes(dst + off, src + off, cnt);
        }
        // The workgroup that copies chunk 0 also copies the scale row
        // (gather.py:86-99, 137-146).
        if (item % nblocks == b)
          copy_bytes(nm.scale_dst + drow * nm.scale_bytes, nm.scale + e * nm.scale_bytes, nm.scale_bytes);
      }
      item += nchunks;
    }
  }
}

__global__ void __launch_bounds__(kThreads) fetch_kernel(const int64_t* todo, int K, int E, const int64_t* row,
                                                         int64_t base, int64_t layer, RingDev r, int64_t* ticket,
                                                         int publish, int wait, int64_t retry_ticks,
                                                         int64_t giveup) {
  if (publish) fetch_publish(todo, K, E, row, base, layer, r, ticket);
  if (wait) {
    __syncthreads();
    fetch_wait(todo, K, r, ticket, retry_ticks, giveup);
  }
}

int g_blocks = 32;
int64_t g_retry_us = 500000;
int64_t g_giveup = 8;

int to_ring(const xp_ring* r, RingDev* out, const char* what) {
  XP_REQUIRE(r && r->req && r->done && r->seq, "%s: ring pointers must be non-null", what);
  XP_REQUIRE(r->block >= 1 && r->ring >= 1, "%s: ring block=%lld ring=%lld", what, (long long)r->block,
             (long long)r->ring);
  *out = RingDev{r->req, r->done, r->seq, r->block, r->ring};
  return XP_OK;
}

}  // namespace
}  // namespace xp

using namespace xp;

extern "C" {

int xp_gather_set_blocks(int blocks) {
  XP_REQUIRE(blocks >= 1 && blocks <= 1024, "xp_gather_set_blocks: %d (1..1024)", blocks);
  g_blocks = blocks;
  return XP_OK;
}

int xp_fetch_set_timing(int64_t retry_us, int64_t giveup) {
  XP_REQUIRE(retry_us >= 1 && giveup >= 0, "xp_fetch_set_timing: retry_us=%lld giveup=%lld", (long long)retry_us,
             (long long)giveup);
  g_retry_us = retry_us;
  g_giveup = giveup;
  return XP_OK;
}

int xp_gather_rows(const int64_t* todo, int64_t K, int64_t num_experts, const int64_t* dst_row,
                   const int64_t* cache_row, const int64_t* src_row, int64_t base, const xp_gather_name* names,
                   int num_names, const int64_t* ssd_todo, int64_t layer, const xp_ring* ring, void* stream) {
  XP_REQUIRE(K >= 0 && K <= (1 << 20), "xp_gather_rows: K=%lld", (long long)K);
  XP_REQUIRE(num_experts >= 1, "xp_gather_rows: num_experts=%lld", (long long)num_experts);
  XP_REQUIRE(num_names >= 1 && num_names <= 2 && names, "xp_gather_rows: %d names (1 or 2)", num_names);
  if (K == 0) return XP_OK;
  XP_REQUIRE(todo && dst_row && cache_row && src_row, "xp_gather_rows: null index tensor");
  GatherArgs a{};
  a.todo = todo;
  a.K = static_cast<int>(K);
  a.E = static_cast<int>(num_experts);
  a.dst_row = dst_row;
  a.cache_row = cache_row;
  a.src_row = src_row;
  a.base = base;
  a.num_names = num_names;
  for (int n = 0; n < num_names; ++n) {
    const xp_gather_name& s = names[n];
    XP_REQUIRE(s.row_bytes > 0 && s.row_bytes % 4 == 0 && s.src_pitch > 0 && s.src_pitch % 4 == 0 &&
                   s.scale_bytes >= 0 && s.scale_bytes % 4 == 0,
               "xp_gather_rows: name %d sizes must be positive multiples of 4 (row %lld, pitch %lld, scale %lld)", n,
               (long long)s.row_bytes, (long long)s.src_pitch, (long long)s.scale_bytes);
    XP_REQUIRE(s.src && s.dst && s.cache && s.scale && s.scale_dst, "xp_gather_rows: name %d has a null buffer", n);
    if (!s.stg)
      XP_REQUIRE(s.src_pitch == s.row_bytes, "xp_gather_rows: uncompressed RAM rows must have the slab's row size");
    a.names[n] = NameDev{static_cast<const uint8_t*>(s.src),
                         s.src_pitch,
                         s.src_rows,
                         static_cast<const uint8_t*>(s.cache),
                         s.cache_rows,
                         static_cast<uint8_t*>(s.dst),
                         s.dst_rows,
                         s.row_bytes,
                         static_cast<uint8_t*>(s.stg),
                         s.stg_rows,
                         static_cast<const uint8_t*>(s.scale),
                         static_cast<uint8_t*>(s.scale_dst),
                         s.scale_bytes};
  }
  int grid = g_blocks;
  if (ring) {
    int rc = to_ring(ring, &a.ring, "xp_gather_rows");
    if (rc) return rc;
    // The copy skips every listed SSD expert, so all of them must be
    // published: the list may not be longer than a ring slot.
    XP_REQUIRE(K <= ring->block, "xp_gather_rows: %lld entries exceed the ring block %lld", (long long)K,
               (long long)ring->block);
    XP_REQUIRE(ssd_todo != nullptr, "xp_gather_rows: a ring needs ssd_todo");
    a.fetch = 1;
    a.ssd = ssd_todo;
    a.layer = layer;
    a.retry_ticks = g_retry_us * wallclock_ticks_per_us();
    a.giveup = g_giveup;
    grid += 1;
  }
  hipLaunchKernelGGL(gather_kernel, dim3(grid), dim3(kThreads), 0, as_stream(stream), a);
  return check_launch("gather_kernel");
}

static int launch_fetch(const int64_t* todo, int64_t K, int64_t E, const int64_t* row, int64_t base, int64_t layer,
                        const xp_ring* ring, int64_t* ticket, int publish, int wait, void* stream,
                        const char* what) {
  XP_REQUIRE(K >= 0 && E >= 1, "%s: K=%lld E=%lld", what, (long long)K, (long long)E);
  if (K == 0) return XP_OK;
  XP_REQUIRE(todo && ticket && (!publish || row), "%s: null argument", what);
  RingDev r;
  int rc = to_ring(ring, &r, what);
  if (rc) return rc;
  // A request slot holds `block` entries: only todo[0 .. min(K, block)) is
  // published and waited on, as the reference's kernels read
  // todo[0 .. BLOCK) (gather.py:216, 254). A prefill chunk's SSD listing is
  // W entries long, but its experts sit at chunk positions below E <= block
  // (table.py:211-216), so nothing listed is dropped.
  if (K > r.block) K = r.block;
  hipLaunchKernelGGL(fetch_kernel, dim3(1), dim3(kThreads), 0, as_stream(stream), todo, static_cast<int>(K),
                     static_cast<int>(E), row, base, layer, r, ticket, publish, wait,
                     g_retry_us * wallclock_ticks_per_us(), g_giveup);
  return check_launch("fetch_kernel");
}

int xp_fetch_rows(const int64_t* todo, int64_t K, int64_t num_experts, const int64_t* row, int64_t base,
                  int64_t layer, const xp_ring* ring, void* stream) {
  // The ticket is the ring's own seq word (gather.py:280-287).
  return launch_fetch(todo, K, num_experts, row, base, layer, ring, ring ? ring->seq : nullptr, 1, 1, stream,
                      "xp_fetch_rows");
}

int xp_fetch_publish_rows(const int64_t* todo, int64_t K, int64_t num_experts, const int64_t* row, int64_t base,
                          int64_t layer, const xp_ring* ring, int64_t* ticket, void* stream) {
  return launch_fetch(todo, K, num_experts, row, base, layer, ring, ticket, 1, 0, stream,
                      "xp_fetch_publish_rows");
}

int xp_fetch_wait_rows(const int64_t* todo, int64_t K, const xp_ring* ring, const int64_t* ticket, void* stream) {
  return launch_fetch(todo, K, 1, nullptr, 0, 0, ring, const_cast<int64_t*>(ticket), 0, 1, stream,
                      "xp_fetch_wait_rows");
}

}  // extern "C"
