// Expert FFN on the slab for the prefill overflow path (and decode):
// fp8 e4m3 weights with 128x128 fp32 block scales, activations quantised to
// fp8 per token and 128-column group, MFMA fp8 grouped GEMMs, fused SiLU*up,
// and the single top-k combine.
//
// The reference hands expert_map to vLLM's fused fp8 MoE and intercepts its
// moe_sum so the top-k sum runs once over all chunks (experts.py:455-604).
// Here every (token, k) pair's expert output is computed independently of
// the other rows of its tile (an MFMA output element depends only on its own
// A row and B column), written once into a persistent buffer, and summed in
// k order in fp32 with one bf16 rounding at the end -- so a chunked run and
// a one-shot run give the same bits.
//
// Numerics of one pair follow the rounding sequence of a w8a8 block-fp8 MoE:
// x -> fp8 per 128-group (scale = max(amax, 1e-10) / 448, q = clamp(x / s));
// h = sum over K blocks of (xq . wq) * (sx * sw) in fp32; gate, up -> bf16;
// a = bf16(bf16(silu(gate)) * up) (silu is returned in bf16 and then
// multiplied, as vLLM's silu_and_mul does); a -> fp8 per 128-group; y
// likewise with w2;
// contribution = bf16(y * routed weight).
//
// Work decomposition: route lists the pairs of each slab slot in CSR form
// and cuts them into tiles of 64 pairs and wide tiles of 128 pairs of one
// slot. At prefill sizes gemm1 and gemm2 run one persistent workgroup per
// CU over (wide tile, column block) items (128 activation columns, 256
// output columns), so each column block of an expert's weights is read
// once, streamed through an LDS ring; for few pairs gemm1 takes 16 rows and 16
// columns of a tile, with the K blocks split over its waves (so a decode
// step of 8 pairs spreads over 256 workgroups), and gemm2 16 rows and 128
// output columns. Launch grids are sized from the shapes alone (bounds on
// the tile counts), so the sequence is graph-capturable; workgroups without
// live work exit at once.
#include <hip/hip_bf16.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace xp {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 64;          // pairs per tile
constexpr int kWM = 2 * kBM;     // pairs per wide tile (the prefill GEMMs' work unit)
constexpr int kBN = 128;         // output columns per workgroup (one quant group for GEMM1)
constexpr int kKB = 128;         // K block = scale block = one MFMA K
constexpr int kThreads = 256;    // 4 waves, split along N (32 columns each)
constexpr int kRouteThreads = 1024;
constexpr int kMaxRouteSlots = 1024;
constexpr float kFp8Max = 448.0f;
constexpr float kEps = 1e-10f;

__device__ __forceinline__ float bf16_round(float v) { return __bfloat162float(__float2bfloat16(v)); }

__device__ __forceinline__ uint32_t bf16_bits(float v) {
  __hip_bfloat16 b = __float2bfloat16(v);
  return static_cast<uint32_t>(*reinterpret_cast<uint16_t*>(&b));
}

__device__ __forceinline__ float bf16_value(uint32_t u16) { return __uint_as_float(u16 << 16); }

// fp32 -> fp8 e4m3 (OCP), round to nearest even; callers clamp to +-448.
__device__ __forceinline__ uint32_t to_fp8(float v) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false)) & 0xffu;
}

__device__ __forceinline__ float quant_scale(float amax) { return fmaxf(amax, kEps) / kFp8Max; }

__device__ __forceinline__ float clamp_fp8(float v) { return fminf(fmaxf(v, -kFp8Max), kFp8Max); }

// a = bf16(bf16(act(g)) * u) for bf16 values g (gate) and u (up): the
// activation in fp32 as vLLM's activation kernels compute it, returned in
// the activation dtype (bf16), then the product of two bf16 values.
// SiLU: g / (1 + exp(-g)); GELU: g * 0.5 * (1 + erf(g / sqrt(2))).
template <int ACT>
__device__ __forceinline__ float act_and_mul(float g, float u) {
  static_assert(ACT == XP_ACT_SILU || ACT == XP_ACT_GELU, "activation");
  float a;
  if constexpr (ACT == XP_ACT_GELU)
    a = g * 0.5f * (1.0f + erff(g * 0.70710678118654752f));
  else
    a = g / (1.0f + expf(-g));
  return bf16_round(bf16_round(a) * u);
}

// The maximum of v over the 16 lanes of its DPP row (lanes 16r .. 16r + 15):
// quad swaps at lane distance 1 and 2, then the half-row and row mirrors,
// each a DPP operand of v_max, with no LDS round trip. Max is exact and
// order-free, so this equals a butterfly over lane distances 1, 2, 4 and 8.
// Every lane of the row must be active.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false)));   // quad [1,0,3,2]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false)));   // quad [2,3,0,1]
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false)));  // row_half_mirror
  return fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false)));  // row_mirror
}

// 16x16 output tile = A[16][128] . B[128][16] in fp8 e4m3. Lane l = 16q + j
// supplies 32 bytes of A row j and of B column j at K offset 32q; the
// instruction maps the bytes of A and B to K in the same way, so the dot
// products are those of the plain layout. Lane l receives C[4q + r][j].
// Zero scale operands select the unscaled instruction.
__device__ __forceinline__ f32x4 mfma_k128(const u32x4 (&a)[2], const u32x4 (&b)[2]) {
  const i32x8 av = {static_cast<int>(a[0].x), static_cast<int>(a[0].y), static_cast<int>(a[0].z),
                    static_cast<int>(a[0].w), static_cast<int>(a[1].x), static_cast<int>(a[1].y),
                    static_cast<int>(a[1].z), static_cast<int>(a[1].w)};
  const i32x8 bv = {static_cast<int>(b[0].x), static_cast<int>(b[0].y), static_cast<int>(b[0].z),
                    static_cast<int>(b[0].w), static_cast<int>(b[1].x), static_cast<int>(b[1].y),
                    static_cast<int>(b[1].z), static_cast<int>(b[1].w)};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, zero, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ void load32(const uint8_t* p, u32x4 (&v)[2]) {
  v[0] = *reinterpret_cast<const u32x4*>(p);
  v[1] = *reinterpret_cast<const u32x4*>(p + 16);
}

// ---- token quantisation: 256 threads per token, 16 lanes per group ----
__device__ __forceinline__ void quant_token(const uint16_t* __restrict__ x, int64_t H, uint8_t* __restrict__ xq,
                                            float* __restrict__ xs, int64_t t, int tid) {
  const uint16_t* row = x + t * H;
  for (int64_t c0 = tid * 8; c0 < H; c0 += 256 * 8) {
    const u32x4 raw = *reinterpret_cast<const u32x4*>(row + c0);
    float v[8];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_value(raw[i] & 0xffffu);
      v[2 * i + 1] = bf16_value(raw[i] >> 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = row16_max(amax);
    const float s = quant_scale(amax);
    uint32_t q0 = 0, q1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q0 |= to_fp8(clamp_fp8(v[i] / s)) << (8 * i);
      q1 |= to_fp8(clamp_fp8(v[4 + i] / s)) << (8 * i);
    }
    *reinterpret_cast<uint2*>(xq + t * H + c0) = make_uint2(q0, q1);
    if ((tid & 15) == 0) xs[t * (H / kKB) + c0 / kKB] = s;
  }
}

__global__ void __launch_bounds__(256) quant_tokens_kernel(const uint16_t* __restrict__ x, int64_t H,
                                                           uint8_t* __restrict__ xq, float* __restrict__ xs) {
  quant_token(x, H, xq, xs, blockIdx.x, threadIdx.x);
}

// Exclusive scan of three counters over a 1024-thread workgroup.
__device__ __forceinline__ int3 block_scan3(int3 v, int3* s_tot, int3* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int3 in = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int ya = __shfl_up(in.x, off, 64), yb = __shfl_up(in.y, off, 64), yc = __shfl_up(in.z, off, 64);
    if (lane >= off) {
      in.x += ya;
      in.y += yb;
      in.z += yc;
    }
  }
  if (lane == 63) s_tot[wave] = in;
  __syncthreads();
  int3 base = make_int3(0, 0, 0), all = make_int3(0, 0, 0);
  for (int w = 0; w < kRouteThreads / 64; ++w) {
    const int3 t = s_tot[w];
    if (w < wave) {
      base.x += t.x;
      base.y += t.y;
      base.z += t.z;
    }
    all.x += t.x;
    all.y += t.y;
    all.z += t.z;
  }
  *total = all;
  return make_int3(base.x + in.x - v.x, base.y + in.y - v.y, base.z + in.z - v.z);
}

// ---- routing: CSR lists of the pairs of each slab slot, and the tiles ----
// offsets[slots + 1]; pairs[offsets[s] .. offsets[s+1]) = pair ids t*topk + k
// of slot s; tiles[0] = live tile count, then (slot, first pair position)
// per tile of kBM pairs; wide[0] = live wide-tile count, then (slot, first
// pair position, pair count) per wide tile of kWM pairs (wide may be null).
// Each wave counts a contiguous range of pairs into its own LDS histogram (no
// contention between waves), so a slot's list is ordered by wave range;
// dynamic LDS = 16 * slots ints.
// Slots of the pairs p0, p0 + 64, ... (kRouteBatch of them; -1 for pairs
// at or past hi, unknown experts and experts without a slot). All id loads
// are issued before the first expert_map load, and all of those before any
// is used, so a batch costs two memory round trips rather than two per pair.
constexpr int kRouteBatch = 16;
__device__ __forceinline__ void route_slots(const void* ids, int eb, int64_t p0, int64_t hi,
                                            const int32_t* __restrict__ expert_map, int E, int slots,
                                            int (&sl)[kRouteBatch]) {
  int64_t e[kRouteBatch];
#pragma unroll
  for (int j = 0; j < kRouteBatch; ++j) {
    const int64_t p = p0 + 64 * j;
    e[j] = p < hi ? load_id(ids, eb, p) : -1;
  }
#pragma unroll
  for (int j = 0; j < kRouteBatch; ++j) sl[j] = (e[j] >= 0 && e[j] < E) ? expert_map[e[j]] : -1;
#pragma unroll
  for (int j = 0; j < kRouteBatch; ++j) sl[j] = sl[j] < slots ? sl[j] : -1;
}

__device__ __forceinline__ void route_block(const void* ids, int eb, int64_t npairs,
                                            const int32_t* __restrict__ expert_map, int E, int slots,
                                            int32_t* __restrict__ offsets, int32_t* __restrict__ pairs,
                                            int32_t* __restrict__ tiles, int32_t* __restrict__ wide, int* s_hist,
                                            int3* s_tot) {
  constexpr int kW = kRouteThreads / 64;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int i = tid; i < kW * slots; i += kRouteThreads) s_hist[i] = 0;
  __syncthreads();
  const int64_t per = (npairs + kW - 1) / kW;
  const int64_t lo = wave * per, hi = lo + per < npairs ? lo + per : npairs;
  int* hist = s_hist + wave * slots;
  // A wave whose range is one batch (up to 16384 pairs in all) keeps its
  // slots in registers for the scatter below instead of loading the ids and
  // expert_map again (two memory round trips).
  const bool one = hi - lo <= 64 * kRouteBatch;
  int sl1[kRouteBatch];
  if (one) {
    route_slots(ids, eb, lo + lane, hi, expert_map, E, slots, sl1);
#pragma unroll
    for (int j = 0; j < kRouteBatch; ++j)
      if (sl1[j] >= 0) atomicAdd(&hist[sl1[j]], 1);
  } else {
    for (int64_t b = lo; b < hi; b += 64 * kRouteBatch) {
      int sl[kRouteBatch];
      route_slots(ids, eb, b + lane, hi, expert_map, E, slots, sl);
#pragma unroll
      for (int j = 0; j < kRouteBatch; ++j)
        if (sl[j] >= 0) atomicAdd(&hist[sl[j]], 1);
    }
  }
  __syncthreads();
  int c = 0;
  if (tid < slots) {
    for (int w = 0; w < kW; ++w) {  // per-wave counts -> per-wave starts within the slot
      const int v = s_hist[w * slots + tid];
      s_hist[w * slots + tid] = c;
      c += v;
    }
  }
  const int nt = (c + kBM - 1) / kBM, nw = (c + kWM - 1) / kWM;
  int3 total;
  const int3 off = block_scan3(make_int3(c, nt, nw), s_tot, &total);
  if (tid < slots) {
    offsets[tid] = off.x;
    for (int w = 0; w < kW; ++w) s_hist[w * slots + tid] += off.x;  // scatter cursors
    for (int i = 0; i < nt; ++i) {
      tiles[1 + 2 * (off.y + i)] = tid;
      tiles[2 + 2 * (off.y + i)] = off.x + i * kBM;
    }
    if (wide)
      for (int i = 0; i < nw; ++i) {
        wide[1 + 3 * (off.z + i)] = tid;
        wide[2 + 3 * (off.z + i)] = off.x + i * kWM;
        wide[3 + 3 * (off.z + i)] = c - i * kWM < kWM ? c - i * kWM : kWM;
      }
  }
  if (tid == 0) {
    offsets[slots] = total.x;
    tiles[0] = total.y;
    if (wide) wide[0] = total.z;
  }
  __syncthreads();
  if (one) {
#pragma unroll
    for (int j = 0; j < kRouteBatch; ++j)
      if (sl1[j] >= 0) pairs[atomicAdd(&hist[sl1[j]], 1)] = static_cast<int32_t>(lo + lane + 64 * j);
    return;
  }
  for (int64_t b = lo; b < hi; b += 64 * kRouteBatch) {
    int sl[kRouteBatch];
    route_slots(ids, eb, b + lane, hi, expert_map, E, slots, sl);
#pragma unroll
    for (int j = 0; j < kRouteBatch; ++j)
      if (sl[j] >= 0) pairs[atomicAdd(&hist[sl[j]], 1)] = static_cast<int32_t>(b + lane + 64 * j);
  }
}

__global__ void __launch_bounds__(kRouteThreads) route_kernel(const void* ids, int eb, int64_t npairs,
                                                              const int32_t* __restrict__ expert_map, int E,
                                                              int slots, int32_t* __restrict__ offsets,
                                                              int32_t* __restrict__ pairs,
                                                              int32_t* __restrict__ tiles,
                                                              int32_t* __restrict__ wide) {
  extern __shared__ int s_hist[];  // [16 waves][slots]
  __shared__ int3 s_tot[kRouteThreads / 64];
  route_block(ids, eb, npairs, expert_map, E, slots, offsets, pairs, tiles, wide, s_hist, s_tot);
}

// Quantisation and routing of one MoE call in one launch: workgroup 0
// routes, workgroup b >= 1 quantises tokens 4(b-1) .. 4(b-1)+3.
__global__ void __launch_bounds__(kRouteThreads) quant_route_kernel(const uint16_t* __restrict__ x, int64_t T,
                                                                    int64_t H, uint8_t* __restrict__ xq,
                                                                    float* __restrict__ xs, const void* ids, int eb,
                                                                    int64_t npairs,
                                                                    const int32_t* __restrict__ expert_map, int E,
                                                                    int slots, int32_t* __restrict__ offsets,
                                                                    int32_t* __restrict__ pairs,
                                                                    int32_t* __restrict__ tiles,
                                                                    int32_t* __restrict__ wide) {
  extern __shared__ int s_hist[];
  __shared__ int3 s_tot[kRouteThreads / 64];
  if (blockIdx.x == 0) {
    route_block(ids, eb, npairs, expert_map, E, slots, offsets, pairs, tiles, wide, s_hist, s_tot);
    return;
  }
  const int64_t t = (static_cast<int64_t>(blockIdx.x) - 1) * 4 + (threadIdx.x >> 8);
  if (t < T) quant_token(x, H, xq, xs, t, threadIdx.x & 255);
}

struct Tile {
  int slot, first, count;
};

// Work item of a 1-D GEMM grid of ncols column blocks per tile, laid out so
// that every column block of a tile runs on the same XCD (workgroup L is
// dispatched to XCD L % 8): the tile's token rows and its expert's weight
// rows are then read into one L2. Tiles t, t + 8, ... belong to XCD t % 8.
__device__ __forceinline__ void xcd_item(int ncols, int& tile, int& col) {
  const int L = blockIdx.x, xcd = L & 7, j = L >> 3;
  tile = (j / ncols) * 8 + xcd;
  col = j - (j / ncols) * ncols;
}

__device__ __forceinline__ bool load_tile_at(int i, const int32_t* tiles, const int32_t* offsets, Tile& t) {
  if (i >= tiles[0]) return false;
  t.slot = tiles[1 + 2 * i];
  t.first = tiles[2 + 2 * i];
  const int end = offsets[t.slot + 1];
  t.count = end - t.first < kBM ? end - t.first : kBM;
  return true;
}

// Prefill-sized calls multiply wide tiles (up to kWM pairs of one slot), so
// that each column block of an expert's weights is read by one workgroup.
// route writes their list after the tile list (wide_list_offset).

// Bounds on the tile and wide-tile counts of npairs pairs over `slots`
// slots (each slot's last tile may be partial).
__host__ __device__ inline int64_t tile_bound(int64_t npairs, int64_t slots) {
  if (npairs <= 0 || slots <= 0) return 0;
  return (npairs + kBM - 1) / kBM + (slots < npairs ? slots : npairs);
}
__host__ __device__ inline int64_t wide_bound(int64_t npairs, int64_t slots) {
  if (npairs <= 0 || slots <= 0) return 0;
  return (npairs + kWM - 1) / kWM + (slots < npairs ? slots : npairs);
}

// The wide-tile list inside the tiles buffer, after the tile list's
// 1 + 2 * tile_bound ints: [0] = count, then (slot, first pair position,
// pair count) per wide tile.
__host__ __device__ inline int64_t wide_list_offset(int64_t npairs, int64_t slots) {
  return 1 + 2 * tile_bound(npairs, slots);
}

// Workspace of xp_moe_experts: bf16 activations, their per-16-column
// maxima, the fp8 activations and their per-128-column scales.
struct Work {
  uint16_t* a16;   // [npairs][I]
  float* amax16;   // [npairs][I/16]
  uint8_t* act;    // [npairs][I]
  float* acts;     // [npairs][I/128]
};

inline int64_t align256(int64_t n) { return (n + 255) & ~int64_t(255); }

inline int64_t work_layout(int64_t npairs, int64_t I, Work* w, uint8_t* base) {
  const int64_t sz[4] = {align256(npairs * I * 2), align256(npairs * (I / 16) * 4), align256(npairs * I),
                         align256(npairs * (I / kKB) * 4)};
  if (w) {
    w->a16 = reinterpret_cast<uint16_t*>(base);
    w->amax16 = reinterpret_cast<float*>(base + sz[0]);
    w->act = base + sz[0] + sz[1];
    w->acts = reinterpret_cast<float*>(base + sz[0] + sz[1] + sz[2]);
  }
  return sz[0] + sz[1] + sz[2] + sz[3];
}

constexpr int kWideTiles = 64;  // tile bound from which gemm1 uses the wide workgroups
constexpr int kNarrowChunk = 4; // K blocks per load chunk of the small-batch GEMMs
constexpr int kMaxKB = 64;    // K blocks a workgroup keeps row scales for (H, I <= 8192)

// ---- prefill GEMMs: persistent workgroups over wide tiles ----
//
// A work item is (wide tile, column block). The items of XCD x belong to the
// wide tiles x, x + 8, x + 16, ..., a tile's column blocks consecutive;
// workgroup b runs on XCD b % 8 and takes that XCD's items l, l + nl,
// l + 2 nl, ... (l = b / 8, nl = gridDim.x / 8), so a tile's column blocks
// run side by side on one XCD and its token rows are read into one L2.
//
// The operands stream through a ring of kRing LDS stages that global-to-LDS
// loads fill without passing through registers: a stage holds one K block
// of the item's weight rows, of the tile's A rows and of the A rows' scales.
// Each wave keeps the loads of the next kRing - 1 blocks in flight while it
// multiplies one, and the stream runs on across items: the next item's rows
// are looked up during the current item's first steps and its first blocks
// are requested during the last, so the epilogue and the next item's set-up
// overlap the loads.
//
// Vector memory operations complete in issue order, so "block k has landed"
// is "at most the loads this wave issued in the last step are in flight"
// (s_waitcnt vmcnt; the count depends on the item, see issue()).
// That holds only if nothing is issued after a step's operand loads, and if
// the compiler adds no waits of its own: every other load in the loop goes
// to LDS or through the scalar cache, and the epilogue's global stores are
// issued at the start of the next item's first step.
constexpr int kRing = 3;
constexpr int kAhead = kRing - 1;  // blocks requested ahead of the one multiplied
constexpr int kRowB = kKB;         // bytes of one operand row's K block (fp8)
constexpr int kGemmWaves = 8;      // waves of a prefill GEMM workgroup
constexpr int kMinSteps = 4;       // steps per item at least (the next item's set-up takes 3)

// This wave's loads but the last N have landed and its LDS writes are done;
// then the workgroup meets. A plain s_barrier: the fence of __syncthreads
// would also wait for the loads in flight.
template <int N>
__device__ __forceinline__ void ring_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// ring_barrier<n> for a wave-uniform n in [lo, hi]: the loads a wave issues
// per step depend on the item (see the prefill GEMMs), so the count left in
// flight is chosen at run time from the immediates the wait takes.
template <int LO, int HI>
__device__ __forceinline__ void ring_barrier_n(int n) {
  if constexpr (LO >= HI) {
    ring_barrier<HI>();
  } else {
    if (n <= LO)
      ring_barrier<LO>();
    else
      ring_barrier_n<LO + 1, HI>(n);
  }
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const void*)p));
}
// A wave-uniform 64-bit address in scalar registers. The readfirstlane
// builtin returns int: each half is taken as uint32_t before widening, or a
// low half with bit 31 set would sign-extend into the high half.
__device__ __forceinline__ uint64_t uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32)));
  return static_cast<uint64_t>(lo) | (static_cast<uint64_t>(hi) << 32);
}
// One piece per lane from global memory into LDS: lane l's 16 (4) bytes, at
// base + off (scalar base, 32-bit vector offset), land at dst + 16 l (4 l);
// base and dst are the same for the whole wave. Written in assembly so that
// the compiler does not track these loads: it would make every LDS access
// wait for all of them. M0 (the LDS destination) is restored afterwards.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, void* dst) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(uniform_ptr(base)), "s"(__builtin_amdgcn_readfirstlane(lds_addr(dst)))
      : "memory");
}
// dma16 marked non-temporal, for weight rows: each is read once per launch,
// so they should not push the activation rows (re-read by every column block
// of a tile) out of the caches. 3-4% off the prefill GEMMs.
__device__ __forceinline__ void dma16_stream(const void* base, uint32_t off, void* dst) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 nt\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(uniform_ptr(base)), "s"(__builtin_amdgcn_readfirstlane(lds_addr(dst)))
      : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, void* dst) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off), "s"(uniform_ptr(base)), "s"(__builtin_amdgcn_readfirstlane(lds_addr(dst)))
      : "memory");
}

// Stage rows are 128 bytes; 16-byte piece p of row r sits at slot p ^ (r & 7),
// so the 8 lanes that read one piece of 8 consecutive rows use distinct
// banks. A load of 8 rows writes slot l & 7 of row l / 8 from lane l, which
// therefore fetches global piece (l & 7) ^ (row & 7).
__device__ __forceinline__ int swizzled_piece(int lane) { return (lane & 7) ^ ((lane >> 3) & 7); }

// A lane's MFMA operand: bytes 32q .. 32q + 31 of stage row `row`.
__device__ __forceinline__ void read_frag(const uint8_t* stage, int row, int q, u32x4 (&v)[2]) {
  const uint8_t* r = stage + row * kRowB;
  const int s = row & 7;
  v[0] = *reinterpret_cast<const u32x4*>(r + (((2 * q) ^ s) << 4));
  v[1] = *reinterpret_cast<const u32x4*>(r + (((2 * q + 1) ^ s) << 4));
}

template <int N>
using Int = std::integral_constant<int, N>;

// Calls f(Int<n>{}) for the tile's subtile count n in 1..kWM/16: the K loop
// is compiled once per count, without branches and with no more
// accumulators than it needs.
template <int N, typename F>
__device__ __forceinline__ void with_subtiles_from(int nmi, F&& f) {
  if constexpr (N >= kWM / 16) {
    f(Int<kWM / 16>{});
  } else {
    if (nmi <= N)
      f(Int<N>{});
    else
      with_subtiles_from<N + 1>(nmi, f);
  }
}

template <typename F>
__device__ __forceinline__ void with_subtiles(int nmi, F&& f) {
  with_subtiles_from<1>(nmi, f);
}

struct Item {
  int slot, first, count, col;  // count 0: no item
};

// Candidate n of this workgroup: item j = l + n * nl of its XCD, i.e. wide
// tile (j / ncols) * 8 + xcd and column block j % ncols. Its list entry is
// read through the scalar cache (the list does not change during the call).
__device__ __forceinline__ Item item_fetch(int n, int ncols, const int32_t* __restrict__ wide, int64_t wmax) {
  const int jj = (static_cast<int>(blockIdx.x) >> 3) + n * (static_cast<int>(gridDim.x) >> 3);
  const int w = __builtin_amdgcn_readfirstlane((jj / ncols) * 8 + (static_cast<int>(blockIdx.x) & 7));
  Item it;
  it.col = __builtin_amdgcn_readfirstlane(jj - (jj / ncols) * ncols);
  it.slot = it.first = it.count = 0;
  const int live = wide[0];
  if (w < live && w < wmax) {
    it.slot = wide[1 + 3 * static_cast<int64_t>(w)];
    it.first = wide[2 + 3 * static_cast<int64_t>(w)];
    it.count = wide[3 + 3 * static_cast<int64_t>(w)];
  }
  return it;
}

// The pairs of an item's rows (padding rows repeat its first pair) into
// s_pn, by waves 0 and 1.
__device__ __forceinline__ void request_pairs(const Item& it, const int32_t* __restrict__ pairs, int* s_pn) {
  const int tid = threadIdx.x, wave = tid >> 6;
  if (wave < kWM / 64) dma4(pairs + it.first, 4 * (tid < it.count ? tid : 0), s_pn + 64 * wave);
}

// s_pair (pair or -1 past the count) and s_row (the operand row, pair / div)
// from s_pn. Pairs are clamped to [0, npairs) before they address anything.
__device__ __forceinline__ void put_rows(const Item& it, const int* s_pn, int div, int64_t npairs, int* s_pair,
                                         int* s_row) {
  const int tid = threadIdx.x;
  if (tid < kWM) {
    const int p = s_pn[tid];
    const int c = p < 0 ? 0 : (p >= npairs ? static_cast<int>(npairs - 1) : p);
    s_pair[tid] = tid < it.count && c == p ? p : -1;
    s_row[tid] = c / div;
  }
}

// Per-lane byte offsets of a wave's A-row and A-scale loads for an item with
// operand rows s_row (A rows of lda bytes, KB scales per row): A stage rows
// 16 wave + 8 i + lane / 8 (i = 0, 1), scale rows 64 (wave & 1) + lane.
struct AOffsets {
  uint32_t a[2];
  uint32_t s;
};

__device__ __forceinline__ AOffsets a_offsets(const int* s_row, int64_t lda, int KB) {
  const int wave = static_cast<int>(threadIdx.x) >> 6, lane = static_cast<int>(threadIdx.x) & 63;
  AOffsets o;
#pragma unroll
  for (int i = 0; i < 2; ++i)
    o.a[i] = static_cast<uint32_t>(s_row[16 * wave + 8 * i + (lane >> 3)] * lda + 16 * swizzled_piece(lane));
  o.s = static_cast<uint32_t>(s_row[64 * (wave & 1) + lane] * KB * 4);
  return o;
}

// GEMM1 at prefill sizes: gate and up for 128 activation columns of a wide
// tile per item; each wave owns 16 columns (16 gate and 16 up rows) and runs
// the K blocks in order, so a column's value does not depend on the
// workgroup width or the tile height. Then a = bf16(bf16(silu(bf16 gate)) *
// bf16 up) is quantised to fp8 per row over the workgroup's 128 columns, one
// scale group. Only the 16-row subtiles that hold pairs are multiplied.
template <int ACT>
__global__ void __launch_bounds__(kGemmWaves * 64) gemm1_kernel(const uint8_t* __restrict__ xq,
                                                               const float* __restrict__ xs, int64_t H, int64_t I,
                                                               int topk, const uint8_t* __restrict__ w13,
                                                               const float* __restrict__ w13_scale,
                                                               const int32_t* __restrict__ pairs,
                                                               const int32_t* __restrict__ wide, int64_t wmax,
                                                               int64_t npairs, Work work) {
  constexpr int NW = kGemmWaves, NT = NW * 64, NC = NW * 16;
  constexpr int NB = 2 * NC;       // weight rows per item: per wave 16 gate, then 16 up
  static_assert(NC == kKB, "a workgroup covers one 128-column scale group of the activations");
  __shared__ __attribute__((aligned(16))) uint8_t s_b[kRing][NB * kRowB];
  __shared__ __attribute__((aligned(16))) uint8_t s_a[kRing][kWM * kRowB];
  __shared__ __attribute__((aligned(16))) float s_s[kRing][kWM];
  __shared__ int s_pn[kWM];
  __shared__ int s_row[2][kWM];
  __shared__ int s_pair[2][kWM];
  __shared__ float s_sw[2][2 * kMaxKB];  // gate (first KB) and up weight scales per K block, two items
  __shared__ float s_m[NW][kWM];         // row maxima per wave (16 columns)
  __shared__ float s_q[kWM];             // row scales of the activations

  const int ncols = static_cast<int>(I / NC);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(H / kKB), KS = KB > kMinSteps ? KB : kMinSteps;

  Item cur = item_fetch(0, ncols, wide, wmax);
  if (cur.count == 0) return;
  Item nxt = item_fetch(1, ncols, wide, wmax);
  int n = 2;

  // Weight-row loads: load i of a wave covers its stage rows 8i .. 8i + 7,
  // gate rows for i < 2 and up rows (I rows further) for i >= 2.
  uint32_t boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    boff[i] = static_cast<uint32_t>(((i >= 2 ? I : 0) + 16 * wave + 8 * (i & 1) + (lane >> 3)) * H +
                                    16 * swizzled_piece(lane));
  auto wbase = [&](const Item& it) {
    return w13 + (static_cast<int64_t>(it.slot) * 2 * I + static_cast<int64_t>(it.col) * NC) * H;
  };
  // Weight scales of an item into s_sw (waves 0 and 1): the workgroup's gate
  // and up rows each lie in one 128-row scale block.
  auto request_weight_scales = [&](const Item& it, float* dst) {
    if (wave < 2) {
      const int i = tid < 2 * KB ? tid : 2 * KB - 1;
      const int64_t blk = static_cast<int64_t>(it.slot) * (2 * I / kKB) + (i < KB ? 0 : I / kKB) + it.col;
      dma4(w13_scale, static_cast<uint32_t>(4 * (blk * KB + (i < KB ? i : i - KB))), dst + 64 * wave);
    }
  };
  // Block kb of an item with nmi live subtiles into `stage`: every wave its
  // 32 weight rows; wave w its A rows 16w .. 16w + 15 only when they hold
  // pairs (w < nmi); waves 0 and 1 the A rows' scales (wave 1's half only
  // when rows 64 and up hold pairs). Returns the loads this wave issued,
  // which the wait before the block after next leaves in flight.
  auto issue = [&](int stage, const uint8_t* wb, const AOffsets& ao, int kb, int nmi) {
    const uint8_t* bsrc = wb + kb * kRowB;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma16_stream(bsrc, boff[i], s_b[stage] + (32 * wave + 8 * i) * kRowB);
    int ops = 4;
    if (wave < nmi) {
      const uint8_t* asrc = xq + kb * kRowB;
#pragma unroll
      for (int i = 0; i < 2; ++i) dma16(asrc, ao.a[i], s_a[stage] + (16 * wave + 8 * i) * kRowB);
      ops += 2;
    }
    if (wave == 0 || (wave == 1 && nmi > 4)) {
      dma4(xs + kb, ao.s, &s_s[stage][64 * wave]);
      ops += 1;
    }
    return ops;
  };
  // The fp8 rows and scales of the previous item, staged in LDS.
  int out_cb = 0, out_c0 = 0, out_rows = 0;
  auto copy_out = [&](const uint8_t* stg) {
    if (tid < out_rows) {
      const int p = s_pair[out_cb][tid];
      if (p >= 0) work.acts[static_cast<int64_t>(p) * (I / kKB) + out_c0 / kKB] = s_q[tid];
    }
    // 16 bytes per thread and pass: 8 threads per row.
    for (int i = tid; i < out_rows * (kKB / 16); i += NT) {
      const int row = i >> 3, piece = i & 7;
      const int p = s_pair[out_cb][row];
      if (p >= 0)
        *reinterpret_cast<u32x4*>(work.act + static_cast<int64_t>(p) * I + out_c0 + piece * 16) =
            *reinterpret_cast<const u32x4*>(stg + row * kRowB + piece * 16);
    }
  };

  request_pairs(cur, pairs, s_pn);
  request_weight_scales(cur, s_sw[0]);
  ring_barrier<0>();
  put_rows(cur, s_pn, topk, npairs, s_pair[0], s_row[0]);
  lds_barrier();
  AOffsets ao_cur = a_offsets(s_row[0], H, KB), ao_nxt = ao_cur;
  issue(0, wbase(cur), ao_cur, 0, (cur.count + 15) >> 4);
  int last_ops = issue(1, wbase(cur), ao_cur, KB > 1 ? 1 : 0, (cur.count + 15) >> 4);

  int st = 0;  // stage of the current step
  int cb = 0;  // row set of the current item
  for (;;) {
    const int nb = cb ^ 1;
    const bool more = nxt.count > 0;
    const uint8_t* wb_cur = wbase(cur);
    const uint8_t* wb_nxt = more ? wbase(nxt) : wb_cur;
    const int nmi = (cur.count + 15) >> 4, nmi_nxt = (nxt.count + 15) >> 4;
    Item after = nxt;

    with_subtiles(nmi, [&](auto nmi_c) {
      constexpr int MI = decltype(nmi_c)::value;
      f32x4 acc[MI][2];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};

      for (int k = 0; k < KS; ++k) {
        ring_barrier_n<4, 7>(last_ops);  // block k is in stage st
        const int sn = st == 0 ? kRing - 1 : st - 1;  // the stage multiplied one step ago
        if (k == 0 && out_rows > 0) {
          copy_out(s_a[sn]);  // staged there by the previous item's epilogue
          out_rows = 0;
          lds_barrier();
        }
        // The next item: its pairs and the entry of the one after (step 0),
        // its rows (1), its A offsets and weight scales (2).
        if (more) {
          if (k == 0) {
            request_pairs(nxt, pairs, s_pn);
            after = item_fetch(n, ncols, wide, wmax);
          } else if (k == 1) {
            put_rows(nxt, s_pn, topk, npairs, s_pair[nb], s_row[nb]);
          } else if (k == 2) {
            ao_nxt = a_offsets(s_row[nb], H, KB);
            request_weight_scales(nxt, s_sw[nb]);
          }
        }
        // Block k + kAhead of this item, or the next item's first blocks.
        const int blk = k + kAhead;
        if (blk < KS || !more)
          last_ops = issue(sn, wb_cur, ao_cur, blk < KB ? blk : KB - 1, nmi);
        else
          last_ops = issue(sn, wb_nxt, ao_nxt, blk - KS < KB ? blk - KS : KB - 1, nmi_nxt);
        if (k < KB) {
          const float g = s_sw[cb][k], u = s_sw[cb][KB + k];
          u32x4 bg[2], bu[2];
          read_frag(s_b[st], 32 * wave + j, q, bg);
          read_frag(s_b[st], 32 * wave + 16 + j, q, bu);
          // Subtile mi + 1's A rows and scales are read while subtile mi
          // multiplies.
          u32x4 a[2][2];
          f32x4 sa[2];
          auto fetch = [&](int mi, int slot) {
            read_frag(s_a[st], 16 * mi + j, q, a[slot]);
            sa[slot] = *reinterpret_cast<const f32x4*>(&s_s[st][16 * mi + 4 * q]);
          };
          fetch(0, 0);
#pragma unroll
          for (int mi = 0; mi < MI; ++mi) {
            const int c = mi & 1;
            if (mi + 1 < MI) fetch(mi + 1, c ^ 1);
            const f32x4 part0 = mfma_k128(a[c], bg), part1 = mfma_k128(a[c], bu);
            // One combined scale per output row and K block (token scale x
            // weight scale), so each MFMA output needs a single FMA.
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              acc[mi][0][r] = fmaf(part0[r], sa[c][r] * g, acc[mi][0][r]);
              acc[mi][1][r] = fmaf(part1[r], sa[c][r] * u, acc[mi][1][r]);
            }
          }
        }
        st = st == kRing - 1 ? 0 : st + 1;
      }

      // 128 columns: one whole scale group of the activations, so they are
      // quantised here (s = max(max |a|, 1e-10) / 448, q = rne(clamp(a / s)),
      // the rule gemm2_narrow_kernel applies, on the same bf16 values). The
      // fp8 rows are staged in the A stage of the last step, which no load
      // targets before the next item's first step writes them out.
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float a = act_and_mul<ACT>(bf16_round(acc[mi][0][r]), bf16_round(acc[mi][1][r]));
          acc[mi][0][r] = a;
          float m = fabsf(a);
          m = row16_max(m);
          if (j == 0) s_m[wave][16 * mi + 4 * q + r] = m;
        }
      }
      lds_barrier();  // s_m; and every wave is done with the last stage
      if (tid < 16 * MI) {
        float m = s_m[0][tid];
#pragma unroll
        for (int w = 1; w < NW; ++w) m = fmaxf(m, s_m[w][tid]);
        s_q[tid] = quant_scale(m);
      }
      lds_barrier();
      uint8_t* stg = s_a[st == 0 ? kRing - 1 : st - 1];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * mi + 4 * q + r;
          stg[row * kRowB + 16 * wave + j] = static_cast<uint8_t>(to_fp8(clamp_fp8(acc[mi][0][r] / s_q[row])));
        }
      }
    });
    out_cb = cb;
    out_c0 = cur.col * NC;
    out_rows = 16 * nmi;
    if (!more) break;
    cur = nxt;
    nxt = after;
    ++n;
    cb = nb;
    ao_cur = ao_nxt;
  }
  lds_barrier();
  copy_out(s_a[st == 0 ? kRing - 1 : st - 1]);
  // The last steps requested blocks that nothing reads: let them land before
  // the workgroup's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Operands of one K block of a 16-row subtile for one wave: the A rows (the
// lane's row j, bytes 32q..32q+31) and two 16-row blocks of B rows.
struct KBlock {
  u32x4 a[2];
  u32x4 b[2][2];
};

// CH consecutive K blocks from kb0, the block index clamped at KB - 1 so
// that the loads are unconditional (a clamped block is loaded, not used).
// The weight rows (B) and the token rows (A) load separately, so that the
// weights can be requested before the tile's rows are looked up.
template <int CH>
__device__ __forceinline__ void load_chunk_b(KBlock (&c)[CH], const uint8_t* const (&brow)[2], int kb0, int KB) {
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int kb = kb0 + i < KB ? kb0 + i : KB - 1;
    load32(brow[0] + kb * kKB, c[i].b[0]);
    load32(brow[1] + kb * kKB, c[i].b[1]);
  }
}

template <int CH>
__device__ __forceinline__ void load_chunk_a(KBlock (&c)[CH], const uint8_t* arow, int kb0, int KB) {
#pragma unroll
  for (int i = 0; i < CH; ++i) load32(arow + (kb0 + i < KB ? kb0 + i : KB - 1) * kKB, c[i].a);
}

template <int CH>
__device__ __forceinline__ void load_chunk(KBlock (&c)[CH], const uint8_t* arow, const uint8_t* const (&brow)[2],
                                           int kb0, int KB) {
  load_chunk_b<CH>(c, brow, kb0, KB);
  load_chunk_a<CH>(c, arow, kb0, KB);
}

// The rows of one 16-row subtile (r0 = its first row in the tile): the
// pair of each row (-1 for padding) and the operand row it reads (padding
// repeats the subtile's first pair).
__device__ __forceinline__ void subtile_rows(const Tile& tile, int r0, const int32_t* pairs, int div, int* s_pair,
                                             int* s_row) {
  const int tid = threadIdx.x;
  if (tid < 16) {
    const int n = tile.count - r0;
    const int p = pairs[tile.first + r0 + (tid < n ? tid : 0)];
    s_pair[tid] = tid < n ? p : -1;
    s_row[tid] = p / div;
  }
}

// GEMM1 for small batches (decode): one 16-row subtile of a tile x 16
// activation columns (gate rows n and up rows I + n) per workgroup. A lone
// subtile is bound by load latency, so the 4 waves split each round of up to
// kSplitRound K blocks, issue all their loads at once and park the raw
// 16x16x128 products in LDS; wave 0 then scales them and sums them in K
// order with one FMA per block and output, the arithmetic of gemm1_kernel,
// so the bits do not depend on the split. 1-D grid in XCD order over
// (subtile, column block) items.
constexpr int kSplitRound = 16;  // K blocks per round, kSplitRound / 4 per wave

template <int ACT>
__global__ void __launch_bounds__(kThreads) gemm1_narrow_kernel(const uint8_t* __restrict__ xq,
                                                                const float* __restrict__ xs, int64_t H, int64_t I,
                                                                int topk, const uint8_t* __restrict__ w13,
                                                                const float* __restrict__ w13_scale,
                                                                const int32_t* __restrict__ offsets,
                                                                const int32_t* __restrict__ pairs,
                                                                const int32_t* __restrict__ tiles, int nsub,
                                                                Work work) {
  constexpr int kPerWave = kSplitRound / (kThreads / 64);
  __shared__ int s_row[16];
  __shared__ int s_pair[16];
  __shared__ float s_xs[16 * kMaxKB];
  __shared__ float s_sw[2][kMaxKB];
  __shared__ float s_m[16];
  __shared__ f32x4 s_part[kSplitRound][2][64];
  __shared__ __attribute__((aligned(16))) uint16_t s_o[16 * 16];

  const int ncb = static_cast<int>(I / 16);
  Tile tile;
  int ti, item;
  xcd_item(nsub * ncb, ti, item);
  if (!load_tile_at(ti, tiles, offsets, tile)) return;
  const int sub = item / ncb, r0 = 16 * sub;
  if (r0 >= tile.count) return;
  const int c0 = (item - sub * ncb) * 16;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(H / kKB);

  // The first round's weight rows depend on the slot alone: request them
  // before the rows and scales are looked up.
  const uint8_t* wslot = w13 + static_cast<int64_t>(tile.slot) * 2 * I * H;
  const int64_t n = c0 + j;
  const uint8_t* const brow[2] = {wslot + n * H + 32 * q, wslot + (I + n) * H + 32 * q};
  const int kw0 = wave * kPerWave;  // this wave's first block of each round, less the round's start
  KBlock c[kPerWave];
  load_chunk_b<kPerWave>(c, brow, kw0, KB);

  subtile_rows(tile, r0, pairs, topk, s_pair, s_row);
  __syncthreads();
  for (int i = tid; i < 16 * KB; i += kThreads) {
    const int r = i / KB, kb = i - r * KB;
    s_xs[i] = xs[static_cast<int64_t>(s_row[r]) * KB + kb];
  }
  {
    const float* sg = w13_scale + (static_cast<int64_t>(tile.slot) * (2 * I / kKB) + c0 / kKB) * KB;
    const float* su = w13_scale + (static_cast<int64_t>(tile.slot) * (2 * I / kKB) + (I + c0) / kKB) * KB;
    for (int i = tid; i < 2 * KB; i += kThreads) s_sw[i / KB][i % KB] = (i < KB ? sg : su)[i % KB];
  }
  const uint8_t* arow = xq + static_cast<int64_t>(s_row[j]) * H + 32 * q;
  load_chunk_a<kPerWave>(c, arow, kw0, KB);
  __syncthreads();  // s_xs, s_sw

  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};  // wave 0's sums
  for (int k0 = 0; k0 < KB; k0 += kSplitRound) {
    const int kw = k0 + kw0;  // this wave's first block of the round
    if (k0 > 0) load_chunk<kPerWave>(c, arow, brow, kw, KB);
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      if (kw + i >= KB) continue;
      s_part[wave * kPerWave + i][0][lane] = mfma_k128(c[i].a, c[i].b[0]);
      s_part[wave * kPerWave + i][1][lane] = mfma_k128(c[i].a, c[i].b[1]);
    }
    __syncthreads();
    if (wave == 0) {
      const int nk = KB - k0 < kSplitRound ? KB - k0 : kSplitRound;
      for (int t = 0; t < nk; ++t) {
        const int kb = k0 + t;
        const float g = s_sw[0][kb], u = s_sw[1][kb];
        const f32x4 pg = s_part[t][0][lane], pu = s_part[t][1][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float sa = s_xs[(4 * q + r) * KB + kb];
          acc[0][r] = fmaf(pg[r], sa * g, acc[0][r]);
          acc[1][r] = fmaf(pu[r], sa * u, acc[1][r]);
        }
      }
    }
    __syncthreads();  // s_part is rewritten by the next round
  }

  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float a = act_and_mul<ACT>(bf16_round(acc[0][r]), bf16_round(acc[1][r]));
      float m = fabsf(a);
      m = row16_max(m);
      const int row = 4 * q + r;
      if (j == 0) s_m[row] = m;
      s_o[row * 16 + j] = static_cast<uint16_t>(bf16_bits(a));
    }
  }
  __syncthreads();
  if (tid < 16) {
    const int p = s_pair[tid];
    if (p >= 0) work.amax16[static_cast<int64_t>(p) * (I / 16) + c0 / 16] = s_m[tid];
  } else if (tid < 48) {  // 16 rows x 2 pieces of 16 bytes
    const int row = (tid - 16) >> 1, piece = tid & 1;
    const int p = s_pair[row];
    if (p >= 0)
      *reinterpret_cast<u32x4*>(work.a16 + static_cast<int64_t>(p) * I + c0 + piece * 8) =
          *reinterpret_cast<const u32x4*>(s_o + row * 16 + piece * 8);
  }
}

// ---- decode steps: two launches for the expert FFN ----
//
// For at most kDecodePairs pairs, every wave of every gemm1 workgroup routes
// the pairs itself (one pair per lane) and the workgroup quantises the token
// rows it multiplies into LDS, so no routing or quantisation launch precedes
// it. gemm2 then takes one token and 8 output columns per workgroup, computes
// each of the token's pairs and sums them there, so no top-k sum launch
// follows. The bits are those of xp_moe_quant_route, xp_moe_experts and
// xp_moe_topk_sum.
constexpr int kDecodePairs = 64;
constexpr int kDecodeMaxH = 4096;       // 16 quantised token rows of H bytes fit in LDS
constexpr int kDecodeActBytes = 32768;  // a token's quantised activations (topk x I) in LDS
constexpr int kDecodeCols2 = 8;         // output columns per gemm2_decode_kernel workgroup

// Pair p's slot (-1: an id outside [0, E) or an expert without a slot):
// from the acquire's per-pair slots when given, else ids then expert_map.
__device__ __forceinline__ int decode_slot(int p, int n, const void* ids, int eb, const int32_t* __restrict__ expert_map,
                                           const int32_t* __restrict__ pair_slot, int E, int slots) {
  const int pc = p < n ? p : 0;  // unconditional loads; lanes past n are not routed
  int sl;
  if (pair_slot) {
    sl = pair_slot[pc];
  } else {
    const int64_t e = load_id(ids, eb, pc);
    sl = e >= 0 && e < E ? expert_map[e] : -1;
  }
  return p < n && sl >= 0 && sl < slots ? sl : -1;
}

// The step's routing as route_kernel lists it (pairs by slot, then by pair
// index; one tile per occupied slot, since a slot holds at most 64 of these
// pairs), computed by one wave from the pairs' slots (lane p: pair p): on
// the lane of each slot's first pair, the slot's 16-row subtiles (nsub) and
// the index of its first one among all the step's subtiles in slot order
// (start); zero subtiles on the other lanes. The loops run over uniform pair
// indices, so each read of another lane's value is a readlane.
struct DecodeRoute {
  int slot, start, nsub;
};

__device__ __forceinline__ DecodeRoute decode_route(int slot, int n) {
  const int lane = threadIdx.x & 63;
  bool first = slot >= 0;
  int count = 0;
  for (int q = 0; q < n; ++q) {
    const int sq = __builtin_amdgcn_readlane(slot, q);
    if (q < lane && sq == slot) first = false;
    count += sq == slot ? 1 : 0;
  }
  const int nsub = first ? (count + 15) >> 4 : 0;
  int start = 0;
  for (int q = 0; q < n; ++q) {
    const int sq = __builtin_amdgcn_readlane(slot, q), nq = __builtin_amdgcn_readlane(nsub, q);
    if (sq < slot) start += nq;
  }
  return DecodeRoute{slot, start, nsub};
}

// gemm1_narrow_kernel over a decode step's pairs, with their routing and the
// quantisation of their token rows done here. Dynamic LDS: 16 x H fp8 rows.
// Every wave routes the step itself (a pair per lane), so the weight rows of
// the workgroup's slot are requested as soon as the pairs' slots arrive; the
// token rows, requested before the slots, are quantised while the weights
// are in flight.
template <int ACT>
__global__ void __launch_bounds__(kThreads) gemm1_decode_kernel(
    const uint16_t* __restrict__ x, int64_t H, int64_t I, const void* ids, int eb, int npairs, int topk,
    const int32_t* __restrict__ expert_map, const int32_t* __restrict__ pair_slot, int E, int slots,
    const uint8_t* __restrict__ w13,
    const float* __restrict__ w13_scale, Work work) {
  constexpr int kPerWave = kSplitRound / (kThreads / 64);
  constexpr int kPre = 4;  // token pieces per thread requested before the routing
  extern __shared__ __attribute__((aligned(16))) uint8_t s_aq[];  // [16][H] fp8 token rows
  __shared__ int s_pair[16];
  __shared__ int s_arow[16];            // LDS row of each subtile row's activations
  __shared__ float s_xs[16 * kMaxKB];   // their scales [LDS row][K block]
  __shared__ float s_sw[2][kMaxKB];
  __shared__ float s_m[16];
  // Raw products of a round: [K block][gate, up][row within the lane's
  // 4-row group][lane], so that a wave reads its own row's values in lane
  // order.
  __shared__ float s_part[kSplitRound][2][4][64];
  __shared__ __attribute__((aligned(16))) uint16_t s_o[16 * 16];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(H / kKB);

  // A token piece (8 columns of token t from column c8) quantised as
  // quant_tokens_kernel does (16 lanes per 128-column group) into LDS row r.
  auto quant_piece = [&](const u32x4& raw, int r, int c8) {
    float v[8];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_value(raw[i] & 0xffffu);
      v[2 * i + 1] = bf16_value(raw[i] >> 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = row16_max(amax);
    const float sc = quant_scale(amax);
    uint32_t q0 = 0, q1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q0 |= to_fp8(clamp_fp8(v[i] / sc)) << (8 * i);
      q1 |= to_fp8(clamp_fp8(v[4 + i] / sc)) << (8 * i);
    }
    *reinterpret_cast<uint2*>(s_aq + r * H + c8) = make_uint2(q0, q1);
    if ((tid & 15) == 0) s_xs[r * KB + c8 / kKB] = sc;
  };
  // With one or two tokens, all their rows are requested before the routing
  // and quantised (piece i of the step: token i / (H / 8)): a batch-1 step
  // is bound by load latency. With more, each workgroup quantises only its
  // subtile's rows once they are known (its pairs are mostly of different
  // tokens, and every token row of the step would be quantised in each of
  // hundreds of workgroups: 143 against 31 us at 8 tokens).
  const int ntok = npairs / topk;
  const bool by_token = ntok <= 2;
  const int nc8 = static_cast<int>(H / 8), npiece = by_token ? ntok * nc8 : 0;
  auto piece_ptr = [&](int i) { return x + static_cast<int64_t>(i / nc8) * H + (i % nc8) * 8; };
  u32x4 xr[kPre];
  if (by_token) {
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int it = tid + kThreads * i;
      xr[i] = *reinterpret_cast<const u32x4*>(piece_ptr(it < npiece ? it : 0));
    }
  }

  const int slot_l = decode_slot(lane, npairs, ids, eb, expert_map, pair_slot, E, slots);
  // gemm2_decode_kernel reads the pairs' slots from the workspace (the
  // activation-scale region, which the decode path does not use).
  if (blockIdx.x == 0 && wave == 0 && lane < npairs) reinterpret_cast<int32_t*>(work.acts)[lane] = slot_l;
  const DecodeRoute rt = decode_route(slot_l, npairs);

  // The workgroup's subtile among all the step's, in slot order, and its
  // column block; the grid bounds the subtiles (the same in every wave).
  const int ncb = static_cast<int>(I / 16);
  int gsi, cbk;
  xcd_item(ncb, gsi, cbk);
  const unsigned long long own = __ballot(rt.nsub > 0 && rt.start <= gsi && gsi < rt.start + rt.nsub);
  if (own == 0) return;
  const int lead = __ffsll(static_cast<long long>(own)) - 1;
  const int slot = __builtin_amdgcn_readlane(slot_l, lead);
  const int sub = gsi - __builtin_amdgcn_readlane(rt.start, lead);
  const unsigned long long mine = __ballot(slot_l == slot);
  const int count = __popcll(mine);
  const int r0 = 16 * sub;  // below count
  const int c0 = cbk * 16;
  const int nrow = count - r0 < 16 ? count - r0 : 16;

  // The slot's gate and up scales, then its weight rows, requested at once.
  const float* sg = w13_scale + (static_cast<int64_t>(slot) * (2 * I / kKB) + c0 / kKB) * KB;
  const float* su = w13_scale + (static_cast<int64_t>(slot) * (2 * I / kKB) + (I + c0) / kKB) * KB;
  const int si = tid < 2 * KB ? tid : 0;
  const float sw = (si < KB ? sg : su)[si < KB ? si : si - KB];
  const uint8_t* wslot = w13 + static_cast<int64_t>(slot) * 2 * I * H;
  const int64_t n = c0 + j;
  const uint8_t* const brow[2] = {wslot + n * H + 32 * q, wslot + (I + n) * H + 32 * q};
  const int kw0 = wave * kPerWave;
  KBlock c[kPerWave];
  load_chunk_b<kPerWave>(c, brow, kw0, KB);

  // Token rows into LDS while the weights are in flight.
  if (by_token) {
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const int it = tid + kThreads * i;
      if (it < npiece) quant_piece(xr[i], it / nc8, (it % nc8) * 8);  // whole 16-lane groups
    }
    for (int it = tid + kThreads * kPre; it < npiece; it += kThreads)
      quant_piece(*reinterpret_cast<const u32x4*>(piece_ptr(it)), it / nc8, (it % nc8) * 8);
  }
  if (tid < 2 * KB) s_sw[tid / KB][tid % KB] = sw;
  // The subtile's rows: the slot's pairs in pair order, rows r0 .. r0 + 15;
  // rows past nrow (outputs not stored) read the subtile's first row.
  if (wave == 0) {
    const int rk = static_cast<int>(lane_prefix(mine));
    const bool in_sub = slot_l == slot && rk >= r0 && rk < r0 + 16;
    const int lead_row = __ffsll(static_cast<long long>(__ballot(slot_l == slot && rk == r0))) - 1;
    if (lane < 16) {
      s_pair[lane] = -1;
      s_arow[lane] = by_token ? lead_row / topk : 0;
    }
    if (in_sub) {
      s_pair[rk - r0] = lane;
      s_arow[rk - r0] = by_token ? lane / topk : rk - r0;
    }
  }
  __syncthreads();  // s_aq, s_xs, s_sw, s_pair, s_arow
  if (!by_token) {
    for (int r = 0; r < nrow; ++r) {
      const uint16_t* row = x + static_cast<int64_t>(s_pair[r] / topk) * H;
      for (int c8 = tid * 8; c8 < H; c8 += kThreads * 8)
        quant_piece(*reinterpret_cast<const u32x4*>(row + c8), r, c8);
    }
    __syncthreads();
  }

  const uint8_t* arow = s_aq + s_arow[j] * H + 32 * q;
  auto load_a = [&](int kb0) {
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const int kb = kb0 + i < KB ? kb0 + i : KB - 1;
      c[i].a[0] = *reinterpret_cast<const u32x4*>(arow + kb * kKB);
      c[i].a[1] = *reinterpret_cast<const u32x4*>(arow + kb * kKB + 16);
    }
  };
  // Wave w scales and sums row 4q + w of the lane's 4-row group (gate and
  // up) in K order, one FMA per block, as gemm1_kernel does.
  const int row = 4 * q + wave;
  const int ar = s_arow[row];
  float acc_g = 0.f, acc_u = 0.f;
  for (int k0 = 0; k0 < KB; k0 += kSplitRound) {
    const int kw = k0 + kw0;
    if (k0 > 0) load_chunk_b<kPerWave>(c, brow, kw, KB);
    load_a(kw);
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      if (kw + i >= KB) continue;
      const f32x4 pg = mfma_k128(c[i].a, c[i].b[0]), pu = mfma_k128(c[i].a, c[i].b[1]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s_part[wave * kPerWave + i][0][r][lane] = pg[r];
        s_part[wave * kPerWave + i][1][r][lane] = pu[r];
      }
    }
    __syncthreads();
    // Row `wave` of the lane's group: fixed offsets from one address, and
    // the whole round unrolled, so every LDS read of the sum is in flight
    // before the FMAs that consume it.
    const float* sp = &s_part[0][0][wave][lane];
    const float* sx = s_xs + ar * KB + k0;
    auto sum_block = [&](int t) {
      const float sa = sx[t];
      acc_g = fmaf(sp[(2 * t) * 256], sa * s_sw[0][k0 + t], acc_g);
      acc_u = fmaf(sp[(2 * t + 1) * 256], sa * s_sw[1][k0 + t], acc_u);
    };
    if (KB - k0 >= kSplitRound) {
#pragma unroll
      for (int t = 0; t < kSplitRound; ++t) sum_block(t);
    } else {
      for (int t = 0; t < KB - k0; ++t) sum_block(t);
    }
    __syncthreads();  // s_part is rewritten by the next round
  }

  {
    const float a = act_and_mul<ACT>(bf16_round(acc_g), bf16_round(acc_u));
    const float m = row16_max(fabsf(a));
    if (j == 0) s_m[row] = m;
    s_o[row * 16 + j] = static_cast<uint16_t>(bf16_bits(a));
  }
  __syncthreads();
  if (tid < 16) {
    const int p = s_pair[tid];
    if (p >= 0) work.amax16[static_cast<int64_t>(p) * (I / 16) + c0 / 16] = s_m[tid];
  } else if (tid < 48) {  // 16 rows x 2 pieces of 16 bytes
    const int rr = (tid - 16) >> 1, piece = tid & 1;
    const int p = s_pair[rr];
    if (p >= 0)
      *reinterpret_cast<u32x4*>(work.a16 + static_cast<int64_t>(p) * I + c0 + piece * 8) =
          *reinterpret_cast<const u32x4*>(s_o + rr * 16 + piece * 8);
  }
}

// gemm2 of a decode step with the top-k sum: one workgroup per (token, 8
// output columns), so that a single token spreads its weight rows over 256
// workgroups; lanes j and j + 8 of the MFMA operand read the same row (one
// request), and columns 8-15 of the product are not used. Its waves take the token's pairs two at a time (wave w:
// pairs w and w + 4, then w + 8 and w + 12, ...); each pair's 16 contributions are computed as
// gemm2_narrow_kernel computes them (the token's quantised activation row as
// every row of the MFMA operand, kNarrowChunk K blocks of weight rows per
// load) and rounded to bf16; then the contributions are summed in k order
// in fp32 and rounded once, as topk_sum_kernel does. A token's experts are
// distinct slots, so its pairs share no weights. The pairs' slots come from
// gemm1_decode_kernel's routing through the workspace, one load instead of
// the ids and expert_map lookups. Pairs whose id is outside [0, E) add
// nothing; so do pairs without a slot (the separate calls would read a
// contribution never written). The slots, the routed weights and the first
// activation pieces are requested first, then each wave's first two pairs'
// weight rows, and the activations are quantised while those are in flight.
__global__ void __launch_bounds__(kThreads) gemm2_decode_kernel(
    int64_t H, int64_t I, int topk, const float* __restrict__ topk_weight, const uint8_t* __restrict__ w2,
    const float* __restrict__ w2_scale, Work work, uint16_t* __restrict__ out) {
  constexpr int NWAVE = kThreads / 64;
  constexpr int kPre = 2;  // activation pieces per thread requested before the weights
  extern __shared__ __attribute__((aligned(16))) uint8_t s_act[];  // [topk][I] fp8 activations
  __shared__ int s_slot[kDecodePairs];
  __shared__ float s_as[kDecodePairs * 4];  // activation scales [pair][K block], K blocks of a round
  __shared__ uint16_t s_c[kDecodePairs][kDecodeCols2];

  const int ncol = static_cast<int>(H / kDecodeCols2);
  const int t = static_cast<int>(blockIdx.x) / ncol;
  const int n0 = (static_cast<int>(blockIdx.x) - t * ncol) * kDecodeCols2;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(I / kKB);
  const int64_t p0 = static_cast<int64_t>(t) * topk;
  const int nc8 = static_cast<int>(I / 8), npiece = topk * nc8;

  // Requests: the pairs' slots as gemm1_decode_kernel routed them (-1: an
  // invalid id or an expert without a slot), the wave's first two pairs'
  // slots and routed weights, and the first activation pieces (8 columns of
  // pair k's bf16 row with the eight 16-column maxima of its group).
  const int32_t* pslot = reinterpret_cast<const int32_t*>(work.acts) + p0;
  const int my_slot = pslot[tid < topk ? tid : 0];
  int kk0[2] = {wave, wave + NWAVE};
  int slot0[2];
  float tw0[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int kc = kk0[h] < topk ? kk0[h] : 0;
    slot0[h] = pslot[kc];
    tw0[h] = topk_weight[p0 + kc];
  }
  auto piece_at = [&](int it, int& k, int& c8) {
    k = it / nc8;
    c8 = (it - k * nc8) * 8;
  };
  u32x4 av[kPre], am[kPre][2];
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const int it = tid + kThreads * i;
    int k, c8;
    piece_at(it < npiece ? it : 0, k, c8);
    const int64_t p = p0 + k;
    av[i] = *reinterpret_cast<const u32x4*>(work.a16 + p * I + c8);
    const float* m = work.amax16 + p * (I / 16) + 8 * (c8 / kKB);
    am[i][0] = *reinterpret_cast<const u32x4*>(m);
    am[i][1] = *reinterpret_cast<const u32x4*>(m + 4);
  }

  // A pair's weight rows for output columns n0 .. n0 + 7 and their scales.
  auto pair_rows = [&](int slot, const uint8_t*& brow, const float*& sw) {
    const int sl = slot < 0 ? 0 : slot;
    brow = w2 + static_cast<int64_t>(sl) * H * I + static_cast<int64_t>(n0 + (j & (kDecodeCols2 - 1))) * I + 32 * q;
    sw = w2_scale + (static_cast<int64_t>(sl) * (H / kKB) + n0 / kKB) * KB;
  };
  // A chunk's weight rows of two pairs, with their K blocks' scales.
  auto load_rows = [&](const int (&slot)[2], const uint8_t* const (&brow)[2], const float* const (&sw)[2], int k0,
                       u32x4 (&b)[2][kNarrowChunk][2], float (&wsc)[2][kNarrowChunk]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (slot[h] < 0) continue;  // uniform
#pragma unroll
      for (int i = 0; i < kNarrowChunk; ++i) {
        const int kb = k0 + i < KB ? k0 + i : KB - 1;
        wsc[h][i] = sw[h][kb];
        load32(brow[h] + kb * kKB, b[h][i]);
      }
    }
  };
#pragma unroll
  for (int h = 0; h < 2; ++h) slot0[h] = kk0[h] < topk ? slot0[h] : -1;
  const uint8_t* brow0[2];
  const float* sw0[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) pair_rows(slot0[h], brow0[h], sw0[h]);
  u32x4 b0[2][kNarrowChunk][2];
  float wsc0[2][kNarrowChunk];
  load_rows(slot0, brow0, sw0, 0, b0, wsc0);

  // The activations quantised into LDS as gemm2_narrow_kernel quantises them
  // (a 128-column group's scale from its eight 16-column maxima).
  auto quant_piece = [&](const u32x4& v, const u32x4 (&mm)[2], int it) {
    int k, c8;
    piece_at(it, k, c8);
    const int g = c8 / kKB;
    float mx = __uint_as_float(mm[0][0]);
#pragma unroll
    for (int u = 1; u < 4; ++u) mx = fmaxf(mx, __uint_as_float(mm[0][u]));
#pragma unroll
    for (int u = 0; u < 4; ++u) mx = fmaxf(mx, __uint_as_float(mm[1][u]));
    const float sc = quant_scale(mx);
    if (c8 % kKB == 0 && g < 4) s_as[k * 4 + g] = sc;
    uint32_t q0 = 0, q1 = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      q0 |= to_fp8(clamp_fp8(bf16_value(v[u] & 0xffffu) / sc)) << (16 * u);
      q0 |= to_fp8(clamp_fp8(bf16_value(v[u] >> 16) / sc)) << (16 * u + 8);
      q1 |= to_fp8(clamp_fp8(bf16_value(v[2 + u] & 0xffffu) / sc)) << (16 * u);
      q1 |= to_fp8(clamp_fp8(bf16_value(v[2 + u] >> 16) / sc)) << (16 * u + 8);
    }
    *reinterpret_cast<uint2*>(s_act + k * I + c8) = make_uint2(q0, q1);
  };
  if (tid < topk) s_slot[tid] = my_slot;
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    const int it = tid + kThreads * i;
    if (it < npiece) quant_piece(av[i], am[i], it);
  }
  for (int it = tid + kThreads * kPre; it < npiece; it += kThreads) {
    int k, c8;
    piece_at(it, k, c8);
    const int64_t p = p0 + k;
    const float* m = work.amax16 + p * (I / 16) + 8 * (c8 / kKB);
    const u32x4 mm[2] = {*reinterpret_cast<const u32x4*>(m), *reinterpret_cast<const u32x4*>(m + 4)};
    quant_piece(*reinterpret_cast<const u32x4*>(work.a16 + p * I + c8), mm, it);
  }
  __syncthreads();

  // One chunk of K blocks of two pairs: their 16 columns scaled and summed
  // in K order in fp32 (row 0 of the product, lanes q = 0, is the pair's
  // value).
  auto mul_chunk = [&](const u32x4 (&b)[2][kNarrowChunk][2], const float (&wsc)[2][kNarrowChunk],
                       const int (&kk)[2], const int (&slot)[2], int k0, float (&acc)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (slot[h] < 0) continue;
      const int64_t p = p0 + kk[h];
      const uint8_t* arow = s_act + kk[h] * I + 32 * q;
      if (k0 + kNarrowChunk <= KB && k0 + kNarrowChunk <= 4) {
        // A whole chunk whose activation scales are all in LDS: every LDS
        // read first, then the products, in K order.
        u32x4 a[kNarrowChunk][2];
        float sa[kNarrowChunk];
#pragma unroll
        for (int i = 0; i < kNarrowChunk; ++i) {
          a[i][0] = *reinterpret_cast<const u32x4*>(arow + (k0 + i) * kKB);
          a[i][1] = *reinterpret_cast<const u32x4*>(arow + (k0 + i) * kKB + 16);
          sa[i] = s_as[kk[h] * 4 + k0 + i];
        }
#pragma unroll
        for (int i = 0; i < kNarrowChunk; ++i) {
          const f32x4 part = mfma_k128(a[i], b[h][i]);
          acc[h] = fmaf(part[0], sa[i] * wsc[h][i], acc[h]);
        }
        continue;
      }
#pragma unroll
      for (int i = 0; i < kNarrowChunk; ++i) {
        const int kb = k0 + i;
        if (kb >= KB) continue;
        u32x4 a[2];
        a[0] = *reinterpret_cast<const u32x4*>(arow + kb * kKB);
        a[1] = *reinterpret_cast<const u32x4*>(arow + kb * kKB + 16);
        // the pair's activation scale for this K block: from LDS for the
        // first four blocks, else recomputed from the maxima
        float sa;
        if (kb < 4) {
          sa = s_as[kk[h] * 4 + kb];
        } else {
          const float* m = work.amax16 + p * (I / 16) + 8 * kb;
          float mx = m[0];
#pragma unroll
          for (int u = 1; u < 8; ++u) mx = fmaxf(mx, m[u]);
          sa = quant_scale(mx);
        }
        const f32x4 part = mfma_k128(a, b[h][i]);
        acc[h] = fmaf(part[0], sa * wsc[h][i], acc[h]);
      }
    }
  };
  auto finish = [&](const int (&kk)[2], const int (&slot)[2], const float (&acc)[2], const float (&tw)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (kk[h] >= topk || q != 0 || j >= kDecodeCols2) continue;
      s_c[kk[h]][j] = slot[h] < 0 ? 0 : static_cast<uint16_t>(bf16_bits(acc[h] * tw[h]));
    }
  };

  // The wave's first two pairs, their first chunk already loaded.
  {
    float acc[2] = {0.f, 0.f};
    mul_chunk(b0, wsc0, kk0, slot0, 0, acc);
    for (int k0 = kNarrowChunk; k0 < KB; k0 += kNarrowChunk) {
      u32x4 b[2][kNarrowChunk][2];
      float wsc[2][kNarrowChunk];
      load_rows(slot0, brow0, sw0, k0, b, wsc);
      mul_chunk(b, wsc, kk0, slot0, k0, acc);
    }
    finish(kk0, slot0, acc, tw0);
  }
  // Further pairs (top-k above 2 x 4 waves), two at a time.
  for (int k = wave + 2 * NWAVE; k < topk; k += 2 * NWAVE) {
    const int kk[2] = {k, k + NWAVE};
    int slot[2];
    float tw[2];
    const uint8_t* brow[2];
    const float* sw[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      slot[h] = kk[h] < topk ? s_slot[kk[h]] : -1;
      tw[h] = kk[h] < topk ? topk_weight[p0 + kk[h]] : 0.f;
      pair_rows(slot[h], brow[h], sw[h]);
    }
    float acc[2] = {0.f, 0.f};
    for (int k0 = 0; k0 < KB; k0 += kNarrowChunk) {
      u32x4 b[2][kNarrowChunk][2];
      float wsc[2][kNarrowChunk];
      load_rows(slot, brow, sw, k0, b, wsc);
      mul_chunk(b, wsc, kk, slot, k0, acc);
    }
    finish(kk, slot, acc, tw);
  }
  __syncthreads();
  if (tid < kDecodeCols2) {
    // The token's contributions in k order, eight LDS reads in flight at a
    // time.
    float sum = 0.f;
    for (int k0 = 0; k0 < topk; k0 += 8) {
      int sl[8];
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u < topk ? k0 + u : topk - 1;
        sl[u] = s_slot[k];
        v[u] = bf16_value(s_c[k][tid]);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u < topk && sl[u] >= 0) sum += v[u];
    }
    out[static_cast<int64_t>(t) * H + n0 + tid] = static_cast<uint16_t>(bf16_bits(sum));
  }
}

// GEMM2 for small batches: one 16-row subtile x 128 output columns (4 waves
// x 32). The subtile's activations arrive as bf16 rows with their
// 16-column maxima (gemm1_narrow_kernel's output): the workgroup quantises
// them itself, with the rule gemm1_kernel applies at prefill sizes, into
// LDS, kQuantK columns per round, and multiplies them from there; the
// weight rows come straight from global memory, CH K blocks per load chunk
// (the first chunk requested before the rows are looked up). Same sums and
// rounding as gemm2_kernel.
constexpr int kQuantK = 2048;  // activation columns quantised per LDS round

template <int CH>
__global__ void __launch_bounds__(kThreads) gemm2_narrow_kernel(int64_t H, int64_t I,
                                                                const float* __restrict__ topk_weight,
                                                                const uint8_t* __restrict__ w2,
                                                                const float* __restrict__ w2_scale,
                                                                const int32_t* __restrict__ offsets,
                                                                const int32_t* __restrict__ pairs,
                                                                const int32_t* __restrict__ tiles, int nsub,
                                                                Work work, uint16_t* __restrict__ out) {
  constexpr int kRoundKB = kQuantK / kKB;
  __shared__ int s_row[16];
  __shared__ int s_pair[16];
  __shared__ float s_as[16 * kMaxKB];
  __shared__ float s_w[16];
  __shared__ float s_sw[kMaxKB];
  __shared__ __attribute__((aligned(16))) uint8_t s_act[16 * kQuantK];
  __shared__ __attribute__((aligned(16))) uint16_t s_o[16 * kBN];

  const int ncb = static_cast<int>(H / kBN);
  Tile tile;
  int ti, item;
  xcd_item(nsub * ncb, ti, item);
  const int sub = item / ncb, cb = item - sub * ncb;
  if (!load_tile_at(ti, tiles, offsets, tile)) return;
  const int r0 = 16 * sub;
  if (r0 >= tile.count) return;
  const int n0 = cb * kBN;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(I / kKB);

  // Weight rows of the first chunk first: they depend on the slot alone.
  const uint8_t* wslot = w2 + static_cast<int64_t>(tile.slot) * H * I;
  const uint8_t* const brow[2] = {wslot + static_cast<int64_t>(n0 + 32 * wave + j) * I + 32 * q,
                                  wslot + static_cast<int64_t>(n0 + 32 * wave + 16 + j) * I + 32 * q};
  KBlock c[CH];
  load_chunk_b<CH>(c, brow, 0, KB);

  subtile_rows(tile, r0, pairs, 1, s_pair, s_row);
  __syncthreads();
  if (tid < 16) s_w[tid] = s_pair[tid] >= 0 ? topk_weight[s_pair[tid]] : 0.f;
  if (tid < KB) s_sw[tid] = w2_scale[(static_cast<int64_t>(tile.slot) * (H / kKB) + n0 / kKB) * KB + tid];

  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  for (int k0 = 0; k0 < KB; k0 += kRoundKB) {
    const int nk = KB - k0 < kRoundKB ? KB - k0 : kRoundKB;
    // Quantise columns [128 k0, 128 (k0 + nk)) of the 16 rows: per row and
    // 128-column group s = max(max |a|, 1e-10) / 448 from the eight
    // 16-column maxima, q = rne(clamp(a / s)); 8 columns per item.
    const int per_row = nk * (kKB / 8);
    for (int i = tid; i < 16 * per_row; i += kThreads) {
      const int r = i / per_row, c8 = (i - r * per_row) * 8, g = k0 + c8 / kKB;
      const int64_t p = s_row[r];
      const float* m = work.amax16 + p * (I / 16) + 8 * g;
      const u32x4 v = *reinterpret_cast<const u32x4*>(work.a16 + p * I + kKB * k0 + c8);
      float mx = m[0];
#pragma unroll
      for (int k = 1; k < 8; ++k) mx = fmaxf(mx, m[k]);
      const float sc = quant_scale(mx);
      if (c8 % kKB == 0) s_as[r * KB + g] = sc;
      uint32_t q0 = 0, q1 = 0;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        q0 |= to_fp8(clamp_fp8(bf16_value(v[k] & 0xffffu) / sc)) << (16 * k);
        q0 |= to_fp8(clamp_fp8(bf16_value(v[k] >> 16) / sc)) << (16 * k + 8);
        q1 |= to_fp8(clamp_fp8(bf16_value(v[2 + k] & 0xffffu) / sc)) << (16 * k);
        q1 |= to_fp8(clamp_fp8(bf16_value(v[2 + k] >> 16) / sc)) << (16 * k + 8);
      }
      *reinterpret_cast<uint2*>(s_act + r * kQuantK + c8) = make_uint2(q0, q1);
    }
    __syncthreads();  // s_act, s_as (and s_w, s_sw)
    for (int kc = 0; kc < nk; kc += CH) {
      if (k0 + kc > 0) load_chunk_b<CH>(c, brow, k0 + kc, KB);
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int kb = k0 + kc + i;
        if (kc + i >= nk) continue;
        const u32x4* pa = reinterpret_cast<const u32x4*>(s_act + j * kQuantK + (kb - k0) * kKB + 32 * q);
        const u32x4 a[2] = {pa[0], pa[1]};
        const float w = s_sw[kb];
        float sc[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[r] = s_as[(4 * q + r) * KB + kb] * w;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const f32x4 part = mfma_k128(a, c[i].b[t]);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[t][r] = fmaf(part[r], sc[r], acc[t][r]);
        }
      }
    }
    __syncthreads();  // the next round rewrites s_act
  }

#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = 4 * q + r;
    const float wgt = s_w[row];
#pragma unroll
    for (int t = 0; t < 2; ++t) s_o[row * kBN + 32 * wave + 16 * t + j] = static_cast<uint16_t>(bf16_bits(acc[t][r] * wgt));
  }
  __syncthreads();
  {  // 16 rows x 16 pieces of 16 bytes: one pass of the 256 threads
    const int row = tid >> 4, col = (tid & 15) * 8;
    const int p = s_pair[row];
    if (p >= 0)
      *reinterpret_cast<u32x4*>(out + static_cast<int64_t>(p) * H + n0 + col) =
          *reinterpret_cast<const u32x4*>(s_o + row * kBN + col);
  }
}

// GEMM2 at prefill sizes: down projection of 128 TB output columns of a wide
// tile per item, times the routed weight, bf16 rows per pair. Each of the 8
// waves owns 16 TB columns and runs the K blocks in order over the tile's
// fp8 activations; persistent over items through the operand ring as
// gemm1_kernel.
template <int TB>
__global__ void __launch_bounds__(kGemmWaves * 64) gemm2_kernel(int64_t H, int64_t I,
                                                               const float* __restrict__ topk_weight,
                                                               const uint8_t* __restrict__ w2,
                                                               const float* __restrict__ w2_scale,
                                                               const int32_t* __restrict__ pairs,
                                                               const int32_t* __restrict__ wide, int64_t wmax,
                                                               int64_t npairs, Work work, uint16_t* __restrict__ out) {
  constexpr int NW = kGemmWaves, NT = NW * 64, NC = NW * 16 * TB;  // output columns per item
  constexpr int kStageRows = 64;  // output rows staged per epilogue round: 64 x NC bf16 = one weight stage
  static_assert(kStageRows * NC * 2 == NC * kRowB, "an epilogue round fills one weight stage");
  __shared__ __attribute__((aligned(16))) uint8_t s_b[kRing][NC * kRowB];
  __shared__ __attribute__((aligned(16))) uint8_t s_a[kRing][kWM * kRowB];
  __shared__ __attribute__((aligned(16))) float s_s[kRing][kWM];
  __shared__ int s_pn[kWM];
  __shared__ int s_row[2][kWM];
  __shared__ int s_pair[2][kWM];
  __shared__ float s_w[2][kWM];
  __shared__ float s_sw[2][2 * kMaxKB];  // weight scales per 128-row block (of TB) and K block, two items

  const int ncols = static_cast<int>(H / NC);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(I / kKB), KS = KB > kMinSteps ? KB : kMinSteps;

  Item cur = item_fetch(0, ncols, wide, wmax);
  if (cur.count == 0) return;
  Item nxt = item_fetch(1, ncols, wide, wmax);
  int n = 2;

  // Weight-row loads: load i of a wave covers its stage rows 8i .. 8i + 7,
  // output columns 16 TB wave + 8i + lane / 8 of the item.
  uint32_t boff[2 * TB];
#pragma unroll
  for (int i = 0; i < 2 * TB; ++i)
    boff[i] = static_cast<uint32_t>((16 * TB * wave + 8 * i + (lane >> 3)) * I + 16 * swizzled_piece(lane));
  auto wbase = [&](const Item& it) {
    return w2 + (static_cast<int64_t>(it.slot) * H + static_cast<int64_t>(it.col) * NC) * I;
  };
  // Weight scales (TB 128-row blocks of w2 x KB) and routed weights of an
  // item into LDS, by waves 0 and 1; the rows s_row must be in place.
  auto request_scales = [&](const Item& it, const int* rows, float* sw, float* wt) {
    if (wave < 2) {
      const int i = tid < TB * KB ? tid : TB * KB - 1;
      const int t = i / KB, kb = i - t * KB;
      dma4(w2_scale, static_cast<uint32_t>(4 * ((static_cast<int64_t>(it.slot) * (H / kKB) + it.col * TB + t) * KB + kb)),
           sw + 64 * wave);
      dma4(topk_weight, static_cast<uint32_t>(4 * rows[tid]), wt + 64 * wave);
    }
  };
  // As gemm1_kernel's: the weight rows always, the A rows of live
  // subtiles, the A scales by waves 0 and 1; returns the loads issued.
  auto issue = [&](int stage, const uint8_t* wb, const AOffsets& ao, int kb, int nmi) {
    const uint8_t* bsrc = wb + kb * kRowB;
#pragma unroll
    for (int i = 0; i < 2 * TB; ++i) dma16_stream(bsrc, boff[i], s_b[stage] + (16 * TB * wave + 8 * i) * kRowB);
    int ops = 2 * TB;
    if (wave < nmi) {
      const uint8_t* asrc = work.act + kb * kRowB;
#pragma unroll
      for (int i = 0; i < 2; ++i) dma16(asrc, ao.a[i], s_a[stage] + (16 * wave + 8 * i) * kRowB);
      ops += 2;
    }
    if (wave == 0 || (wave == 1 && nmi > 4)) {
      dma4(work.acts + kb, ao.s, &s_s[stage][64 * wave]);
      ops += 1;
    }
    return ops;
  };
  // Output rows [r0, r0 + rows) of an item, staged in LDS.
  int out_cb = 0, out_n0 = 0, out_r0 = 0, out_rows = 0;
  auto copy_out = [&](const uint16_t* stg) {
    for (int i = tid; i < out_rows * (NC / 8); i += NT) {
      const int rr = i / (NC / 8), piece = i - rr * (NC / 8);
      const int p = s_pair[out_cb][out_r0 + rr];
      *reinterpret_cast<u32x4*>(out + static_cast<int64_t>(p) * H + out_n0 + piece * 8) =
          *reinterpret_cast<const u32x4*>(stg + rr * NC + piece * 8);
    }
  };

  request_pairs(cur, pairs, s_pn);
  ring_barrier<0>();
  put_rows(cur, s_pn, 1, npairs, s_pair[0], s_row[0]);
  lds_barrier();
  request_scales(cur, s_row[0], s_sw[0], s_w[0]);
  AOffsets ao_cur = a_offsets(s_row[0], I, KB), ao_nxt = ao_cur;
  ring_barrier<0>();
  issue(0, wbase(cur), ao_cur, 0, (cur.count + 15) >> 4);
  int last_ops = issue(1, wbase(cur), ao_cur, KB > 1 ? 1 : 0, (cur.count + 15) >> 4);

  int st = 0;
  int cb = 0;
  for (;;) {
    const int nb = cb ^ 1;
    const bool more = nxt.count > 0;
    const uint8_t* wb_cur = wbase(cur);
    const uint8_t* wb_nxt = more ? wbase(nxt) : wb_cur;
    const int nmi = (cur.count + 15) >> 4, nmi_nxt = (nxt.count + 15) >> 4;
    const int n0 = cur.col * NC;
    Item after = nxt;

    with_subtiles(nmi, [&](auto nmi_c) {
      constexpr int MI = decltype(nmi_c)::value;
      f32x4 acc[MI][TB];
#pragma unroll
      for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int t = 0; t < TB; ++t) acc[mi][t] = f32x4{0.f, 0.f, 0.f, 0.f};

      for (int k = 0; k < KS; ++k) {
        ring_barrier_n<2 * TB, 2 * TB + 3>(last_ops);
        const int sn = st == 0 ? kRing - 1 : st - 1;
        if (k == 0 && out_rows > 0) {
          copy_out(reinterpret_cast<const uint16_t*>(s_b[sn]));
          out_rows = 0;
          lds_barrier();
        }
        if (more) {
          if (k == 0) {
            request_pairs(nxt, pairs, s_pn);
            after = item_fetch(n, ncols, wide, wmax);
          } else if (k == 1) {
            put_rows(nxt, s_pn, 1, npairs, s_pair[nb], s_row[nb]);
          } else if (k == 2) {
            ao_nxt = a_offsets(s_row[nb], I, KB);
            request_scales(nxt, s_row[nb], s_sw[nb], s_w[nb]);
          }
        }
        const int blk = k + kAhead;
        if (blk < KS || !more)
          last_ops = issue(sn, wb_cur, ao_cur, blk < KB ? blk : KB - 1, nmi);
        else
          last_ops = issue(sn, wb_nxt, ao_nxt, blk - KS < KB ? blk - KS : KB - 1, nmi_nxt);
        if (k < KB) {
          const float w = s_sw[cb][(TB * wave / 8) * KB + k];
          u32x4 b[TB][2];
#pragma unroll
          for (int t = 0; t < TB; ++t) read_frag(s_b[st], 16 * TB * wave + 16 * t + j, q, b[t]);
          u32x4 a[2][2];
          f32x4 sa[2];
          auto fetch = [&](int mi, int slot) {
            read_frag(s_a[st], 16 * mi + j, q, a[slot]);
            sa[slot] = *reinterpret_cast<const f32x4*>(&s_s[st][16 * mi + 4 * q]);
          };
          fetch(0, 0);
#pragma unroll
          for (int mi = 0; mi < MI; ++mi) {
            const int c = mi & 1;
            if (mi + 1 < MI) fetch(mi + 1, c ^ 1);
#pragma unroll
            for (int t = 0; t < TB; ++t) {
              const f32x4 part = mfma_k128(a[c], b[t]);
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[mi][t][r] = fmaf(part[r], sa[c][r] * w, acc[mi][t][r]);
            }
          }
        }
        st = st == kRing - 1 ? 0 : st + 1;
      }

      // bf16(acc x routed weight), staged 64 rows at a time in the weight
      // stage of the last step (no load targets it before the next item's
      // first step); the last round is written out at that step.
      uint16_t* stg = reinterpret_cast<uint16_t*>(s_b[st == 0 ? kRing - 1 : st - 1]);
      constexpr int kRounds = (MI + kStageRows / 16 - 1) / (kStageRows / 16);
#pragma unroll
      for (int rd = 0; rd < kRounds; ++rd) {
        const int r0 = rd * kStageRows;
        if (rd > 0) {  // an earlier round: written out now
          lds_barrier();
          copy_out(stg);
        }
        lds_barrier();  // every wave is done with the last stage, or with the previous round
#pragma unroll
        for (int mi = rd * (kStageRows / 16); mi < MI && mi < (rd + 1) * (kStageRows / 16); ++mi) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = 16 * mi + 4 * q + r;
            const float wgt = s_w[cb][row];
#pragma unroll
            for (int t = 0; t < TB; ++t)
              stg[(row - r0) * NC + 16 * TB * wave + 16 * t + j] = static_cast<uint16_t>(bf16_bits(acc[mi][t][r] * wgt));
          }
        }
        out_cb = cb;
        out_n0 = n0;
        out_r0 = r0;
        out_rows = cur.count - r0 < kStageRows ? cur.count - r0 : kStageRows;
      }
    });
    if (!more) break;
    cur = nxt;
    nxt = after;
    ++n;
    cb = nb;
    ao_cur = ao_nxt;
  }
  lds_barrier();
  copy_out(reinterpret_cast<const uint16_t*>(s_b[st == 0 ? kRing - 1 : st - 1]));
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// out[t] = bf16(sum over k of contrib[t*topk + k]) in fp32, k ascending,
// over the pairs whose id is a valid expert.
template <typename Id>
__global__ void __launch_bounds__(256) topk_sum_kernel(const uint16_t* __restrict__ contrib, int64_t H, int topk,
                                                       const Id* __restrict__ ids, int E, uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.y;
  const int64_t c = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 8;
  if (c >= H) return;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // Eight pairs at a time: the ids and the contribution rows are loaded
  // together (a row is read whatever its id, and skipped in the sum), so
  // the loads do not wait on one another.
  for (int k0 = 0; k0 < topk; k0 += 8) {
    bool ok[8];
    u32x4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = k0 + i < topk ? k0 + i : topk - 1;
      const int64_t p = t * topk + k;
      const int64_t e = ids[p];
      ok[i] = k0 + i < topk && e >= 0 && e < E;
      v[i] = *reinterpret_cast<const u32x4*>(contrib + p * H + c);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (!ok[i]) continue;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        s[2 * w] += bf16_value(v[i][w] & 0xffffu);
        s[2 * w + 1] += bf16_value(v[i][w] >> 16);
      }
    }
  }
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = bf16_bits(s[2 * i]) | (bf16_bits(s[2 * i + 1]) << 16);
  *reinterpret_cast<u32x4*>(out + t * H + c) = o;
}

}  // namespace
}  // namespace xp

using namespace xp;

extern "C" {

int64_t xp_moe_max_tiles(int64_t npairs, int64_t slots) {
  if (npairs <= 0 || slots <= 0) return 0;
  // The tile list, then the wide-tile list (1 + 3 * wide_bound ints), in
  // two-int entries past tiles[0].
  return tile_bound(npairs, slots) + (2 + 3 * wide_bound(npairs, slots)) / 2;
}

int xp_quant_tokens(const uint16_t* x, int64_t T, int64_t H, uint8_t* xq, float* xs, void* stream) {
  XP_REQUIRE(T >= 0 && T <= INT32_MAX && H > 0 && H % kKB == 0,
             "xp_quant_tokens: T=%lld, H=%lld (H must be a positive multiple of %d)", (long long)T, (long long)H,
             kKB);
  if (T == 0) return XP_OK;
  XP_REQUIRE(x && xq && xs && aligned16(x) && aligned16(xq), "xp_quant_tokens: null or misaligned buffer");
  hipLaunchKernelGGL(quant_tokens_kernel, dim3(static_cast<unsigned>(T)), dim3(256), 0, as_stream(stream), x, H, xq,
                     xs);
  return check_launch("quant_tokens_kernel");
}

int xp_moe_route(const void* topk_ids, int topk_elem_bytes, int64_t T, int64_t topk, const int32_t* expert_map,
                 int64_t num_experts, int64_t slots, int32_t* offsets, int32_t* pairs, int32_t* tiles, void* stream) {
  XP_REQUIRE(topk_elem_bytes == 4 || topk_elem_bytes == 8, "xp_moe_route: id size %d", topk_elem_bytes);
  XP_REQUIRE(T >= 0 && topk >= 1 && T * topk <= INT32_MAX, "xp_moe_route: T=%lld, topk=%lld", (long long)T,
             (long long)topk);
  XP_REQUIRE(slots >= 1 && slots <= kMaxRouteSlots, "xp_moe_route: %lld slots (at most %d)", (long long)slots,
             kMaxRouteSlots);
  XP_REQUIRE(num_experts >= 1 && num_experts <= INT32_MAX, "xp_moe_route: %lld experts", (long long)num_experts);
  XP_REQUIRE(expert_map && offsets && pairs && tiles && (T == 0 || topk_ids), "xp_moe_route: null argument");
  const size_t lds = static_cast<size_t>(kRouteThreads / 64) * static_cast<size_t>(slots) * sizeof(int);
  int32_t* wide = T * topk > 0 ? tiles + wide_list_offset(T * topk, slots) : nullptr;
  hipLaunchKernelGGL(route_kernel, dim3(1), dim3(kRouteThreads), lds, as_stream(stream), topk_ids, topk_elem_bytes,
                     T * topk, expert_map, static_cast<int>(num_experts), static_cast<int>(slots), offsets, pairs,
                     tiles, wide);
  return check_launch("route_kernel");
}

int xp_moe_quant_route(const uint16_t* x, int64_t T, int64_t H, uint8_t* xq, float* xs, const void* topk_ids,
                       int topk_elem_bytes, int64_t topk, const int32_t* expert_map, int64_t num_experts,
                       int64_t slots, int32_t* offsets, int32_t* pairs, int32_t* tiles, void* stream) {
  XP_REQUIRE(T >= 0 && T <= INT32_MAX && H > 0 && H % kKB == 0,
             "xp_moe_quant_route: T=%lld, H=%lld (H must be a positive multiple of %d)", (long long)T,
             (long long)H, kKB);
  XP_REQUIRE(topk_elem_bytes == 4 || topk_elem_bytes == 8, "xp_moe_quant_route: id size %d", topk_elem_bytes);
  XP_REQUIRE(topk >= 1 && T * topk <= INT32_MAX, "xp_moe_quant_route: topk=%lld", (long long)topk);
  XP_REQUIRE(slots >= 1 && slots <= kMaxRouteSlots, "xp_moe_quant_route: %lld slots (at most %d)",
             (long long)slots, kMaxRouteSlots);
  XP_REQUIRE(num_experts >= 1 && num_experts <= INT32_MAX, "xp_moe_quant_route: %lld experts",
             (long long)num_experts);
  XP_REQUIRE(expert_map && offsets && pairs && tiles, "xp_moe_quant_route: null argument");
  XP_REQUIRE(T == 0 || (x && xq && xs && topk_ids && aligned16(x) && aligned16(xq)),
             "xp_moe_quant_route: null or misaligned buffer");
  const size_t lds = static_cast<size_t>(kRouteThreads / 64) * static_cast<size_t>(slots) * sizeof(int);
  const unsigned grid = static_cast<unsigned>(1 + (T + 3) / 4);
  int32_t* wide = T * topk > 0 ? tiles + wide_list_offset(T * topk, slots) : nullptr;
  hipLaunchKernelGGL(quant_route_kernel, dim3(grid), dim3(kRouteThreads), lds, as_stream(stream), x, T, H, xq, xs,
                     topk_ids, topk_elem_bytes, T * topk, expert_map, static_cast<int>(num_experts),
                     static_cast<int>(slots), offsets, pairs, tiles, wide);
  return check_launch("quant_route_kernel");
}

int64_t xp_moe_workspace_bytes(int64_t npairs, int64_t I) {
  if (npairs <= 0 || I <= 0) return 0;
  return work_layout(npairs, I, nullptr, nullptr);
}

}  // extern "C"

namespace xp {
namespace {

// Argument checks shared by the expert entry points (all but the
// workspace's and the token operands').
int check_ffn(const char* what, int64_t T, int64_t topk, const float* topk_weight, int64_t H, int64_t I,
              const uint8_t* w13, const float* w13_scale, const uint8_t* w2, const float* w2_scale, int64_t slots,
              const int32_t* offsets, const int32_t* pairs, const int32_t* tiles, const uint16_t* out) {
  XP_REQUIRE(H > 0 && I > 0 && H % kBN == 0 && I % kBN == 0 && H <= kKB * kMaxKB && I <= kKB * kMaxKB,
             "%s: H=%lld and I=%lld must be multiples of %d, at most %d", what, (long long)H, (long long)I, kBN,
             kKB * kMaxKB);
  XP_REQUIRE(T >= 0 && topk >= 1 && T * topk <= INT32_MAX && slots >= 1 && slots <= kMaxRouteSlots,
             "%s: T=%lld, topk=%lld, slots=%lld", what, (long long)T, (long long)topk, (long long)slots);
  if (T == 0) return XP_OK;
  XP_REQUIRE(topk_weight && w13 && w13_scale && w2 && w2_scale && offsets && pairs && tiles && out,
             "%s: null argument", what);
  XP_REQUIRE(aligned16(w13) && aligned16(w2) && aligned16(out), "%s: fp8 and output buffers must be 16-byte aligned",
             what);
  const int64_t bound = tile_bound(T * topk, slots);
  XP_REQUIRE(bound <= 65535, "%s: %lld tiles exceed the launch grid", what, (long long)bound);
  return XP_OK;
}

int check_experts(const char* what, const uint8_t* xq, const float* xs, int64_t T, int64_t topk,
                  const float* topk_weight, int64_t H, int64_t I, const uint8_t* w13, const float* w13_scale,
                  const uint8_t* w2, const float* w2_scale, int64_t slots, const int32_t* offsets,
                  const int32_t* pairs, const int32_t* tiles, const uint16_t* out, int activation) {
  XP_REQUIRE(activation == XP_ACT_SILU || activation == XP_ACT_GELU, "%s: unknown activation %d", what, activation);
  const int rc = check_ffn(what, T, topk, topk_weight, H, I, w13, w13_scale, w2, w2_scale, slots, offsets, pairs,
                           tiles, out);
  if (rc || T == 0) return rc;
  XP_REQUIRE(xq && xs && aligned16(xq), "%s: xq and xs must be non-null, xq 16-byte aligned", what);
  return XP_OK;
}

// Compute units per XCD of the current device (8 XCDs), looked up once per
// device.
int cus_per_xcd(int* out) {
  static std::mutex mu;
  static int cache[64];
  int dev = -1;
  XP_HIP(hipGetDevice(&dev));
  XP_REQUIRE(dev >= 0 && dev < 64, "device %d (at most 64 devices)", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int n = 0;
    XP_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
    cache[dev] = n / 8 > 0 ? n / 8 : 1;
  }
  *out = cache[dev];
  return XP_OK;
}

// The two (or, for few pairs, narrow) GEMM launches of one expert call over a
// workspace of xp_moe_workspace_bytes(T * topk, I) bytes at `work`.
int launch_experts(const uint8_t* xq, const float* xs, int64_t T, int64_t topk, const float* topk_weight, int64_t H,
                   int64_t I, const uint8_t* w13, const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                   int64_t slots, const int32_t* offsets, const int32_t* pairs, const int32_t* tiles, uint8_t* work,
                   uint16_t* out, int act, void* stream) {
  const int64_t npairs = T * topk;
  const int64_t bound = tile_bound(npairs, slots);
  Work w;
  work_layout(npairs, I, &w, work);
  // Prefill-sized calls run persistent workgroups over wide tiles, 128
  // activation (gemm1) or output (gemm2) columns per item, and quantise the
  // activations in gemm1; small calls take 16-row subtiles (more workgroups
  // for few pairs) and the small-batch gemm2 quantises. Every column is
  // computed the same way in both.
  const bool narrow = bound < kWideTiles;
  int rc = XP_OK;
  if (!narrow) {
    XP_REQUIRE(T * H <= UINT32_MAX && npairs * I <= UINT32_MAX,
               "xp_moe_experts: T*H=%lld and T*topk*I=%lld must stay below 2^32 (call over fewer tokens)",
               (long long)(T * H), (long long)(npairs * I));
    int per_xcd = 0;
    rc = cus_per_xcd(&per_xcd);
    if (rc) return rc;
    const int64_t wmax = wide_bound(npairs, slots);
    const int32_t* wide = tiles + wide_list_offset(npairs, slots);
    const int64_t per_xcd_tiles = (wmax + 7) / 8;  // wide tiles of one XCD, at most
    // One workgroup per CU: the operand ring takes most of its LDS.
    const int64_t n1 = std::min<int64_t>(per_xcd, per_xcd_tiles * (I / (16 * kGemmWaves)));
    if (act == XP_ACT_GELU)
      hipLaunchKernelGGL(gemm1_kernel<XP_ACT_GELU>, dim3(static_cast<unsigned>(8 * n1)), dim3(64 * kGemmWaves), 0,
                         as_stream(stream), xq, xs, H, I, static_cast<int>(topk), w13, w13_scale, pairs, wide, wmax,
                         npairs, w);
    else
      hipLaunchKernelGGL(gemm1_kernel<XP_ACT_SILU>, dim3(static_cast<unsigned>(8 * n1)), dim3(64 * kGemmWaves), 0,
                         as_stream(stream), xq, xs, H, I, static_cast<int>(topk), w13, w13_scale, pairs, wide, wmax,
                         npairs, w);
    rc = check_launch("gemm1_kernel");
    if (rc) return rc;
    // 256 output columns per item where H allows, else 128.
    if (H % (2 * kBN) == 0) {
      const int64_t n2 = std::min<int64_t>(per_xcd, per_xcd_tiles * (H / (2 * kBN)));
      hipLaunchKernelGGL(gemm2_kernel<2>, dim3(static_cast<unsigned>(8 * n2)), dim3(64 * kGemmWaves), 0,
                         as_stream(stream), H, I, topk_weight, w2, w2_scale, pairs, wide, wmax, npairs, w, out);
    } else {
      const int64_t n2 = std::min<int64_t>(per_xcd, per_xcd_tiles * (H / kBN));
      hipLaunchKernelGGL(gemm2_kernel<1>, dim3(static_cast<unsigned>(8 * n2)), dim3(64 * kGemmWaves), 0,
                         as_stream(stream), H, I, topk_weight, w2, w2_scale, pairs, wide, wmax, npairs, w, out);
    }
    return check_launch("gemm2_kernel");
  }
  const int64_t tiles8 = (bound + 7) / 8 * 8;  // the XCD-aware grids cover whole groups of 8 tiles
  const int64_t g2 = tiles8 * (H / kBN);
  // 16-row subtiles a tile can have: a tile holds at most min(64, npairs) pairs.
  const int nsub = static_cast<int>(((npairs < kBM ? npairs : kBM) + 15) / 16);
  // Few pairs: 16-row subtiles x 16 columns, the K blocks split over 4 waves.
  const int64_t g1n = tiles8 * nsub * (I / 16);
  XP_REQUIRE(g1n <= INT32_MAX && nsub * g2 <= INT32_MAX, "xp_moe_experts: grid too large");
  if (act == XP_ACT_GELU)
    hipLaunchKernelGGL(gemm1_narrow_kernel<XP_ACT_GELU>, dim3(static_cast<unsigned>(g1n)), dim3(kThreads), 0,
                       as_stream(stream), xq, xs, H, I, static_cast<int>(topk), w13, w13_scale, offsets, pairs, tiles,
                       nsub, w);
  else
    hipLaunchKernelGGL(gemm1_narrow_kernel<XP_ACT_SILU>, dim3(static_cast<unsigned>(g1n)), dim3(kThreads), 0,
                       as_stream(stream), xq, xs, H, I, static_cast<int>(topk), w13, w13_scale, offsets, pairs, tiles,
                       nsub, w);
  rc = check_launch("gemm1_narrow_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(gemm2_narrow_kernel<kNarrowChunk>, dim3(static_cast<unsigned>(nsub * g2)), dim3(kThreads), 0,
                     as_stream(stream), H, I, topk_weight, w2, w2_scale, offsets, pairs, tiles, nsub, w, out);
  return check_launch("gemm2_narrow_kernel");
}

}  // namespace
}  // namespace xp

extern "C" {

int xp_moe_experts(const uint8_t* xq, const float* xs, int64_t T, int64_t topk, const float* topk_weight, int64_t H,
                   int64_t I, const uint8_t* w13, const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                   int64_t slots, const int32_t* offsets, const int32_t* pairs, const int32_t* tiles, void* work,
                   int64_t work_bytes, uint16_t* out, int activation, void* stream) {
  int rc = check_experts("xp_moe_experts", xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2, w2_scale, slots,
                         offsets, pairs, tiles, out, activation);
  if (rc || T == 0) return rc;
  XP_REQUIRE(work && (reinterpret_cast<uintptr_t>(work) & 255) == 0,
             "xp_moe_experts: the workspace must be non-null and 256-byte aligned");
  const int64_t need = xp_moe_workspace_bytes(T * topk, I);
  XP_REQUIRE(work_bytes >= need, "xp_moe_experts: workspace of %lld B, needs %lld", (long long)work_bytes,
             (long long)need);
  return launch_experts(xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2, w2_scale, slots, offsets, pairs,
                        tiles, static_cast<uint8_t*>(work), out, activation, stream);
}

int xp_moe_experts_noalloc(const uint8_t* xq, const float* xs, int64_t T, int64_t topk, const float* topk_weight,
                           int64_t H, int64_t I, const uint8_t* w13, const float* w13_scale, const uint8_t* w2,
                           const float* w2_scale, int64_t slots, const int32_t* offsets, const int32_t* pairs,
                           const int32_t* tiles, uint16_t* out, int activation, void* stream) {
  int rc = check_experts("xp_moe_experts_noalloc", xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2,
                         w2_scale, slots, offsets, pairs, tiles, out, activation);
  if (rc || T == 0) return rc;
  const int64_t need = xp_moe_workspace_bytes(T * topk, I);
  if (need > XP_MOE_SCRATCH_BYTES)
    return fail(XP_E_LIMIT,
                "xp_moe_experts_noalloc: %lld pairs x I=%lld need a workspace of %lld B, above the library's "
                "%lld B; call xp_moe_experts with a workspace instead",
                (long long)(T * topk), (long long)I, (long long)need, (long long)XP_MOE_SCRATCH_BYTES);
  uint8_t* work = nullptr;
  rc = moe_scratch_address(&work);
  if (rc) return rc;
  return launch_experts(xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2, w2_scale, slots, offsets, pairs,
                        tiles, work, out, activation, stream);
}

int xp_moe_decode_experts(const uint16_t* x, int64_t T, int64_t H, const void* topk_ids, int topk_elem_bytes,
                          int64_t topk, const float* topk_weight, const int32_t* expert_map,
                          const int32_t* pair_slot, int64_t num_experts, int64_t I, const uint8_t* w13,
                          const float* w13_scale, const uint8_t* w2, const float* w2_scale, int64_t slots, void* work,
                          int64_t work_bytes, uint16_t* out, int activation, void* stream) {
  const char* what = "xp_moe_decode_experts";
  XP_REQUIRE(T >= 0 && topk >= 1 && T * topk <= INT32_MAX, "%s: T=%lld, topk=%lld", what, (long long)T,
             (long long)topk);
  if (T == 0) return XP_OK;
  const int64_t npairs = T * topk;
  if (npairs > kDecodePairs || H > kDecodeMaxH || topk * I > kDecodeActBytes)
    return fail(XP_E_LIMIT,
                "%s: %lld pairs (at most %d), H=%lld (at most %d), topk*I=%lld (at most %d): use the separate calls",
                what, (long long)npairs, kDecodePairs, (long long)H, kDecodeMaxH, (long long)(topk * I),
                kDecodeActBytes);
  XP_REQUIRE(topk_elem_bytes == 4 || topk_elem_bytes == 8, "%s: id size %d", what, topk_elem_bytes);
  XP_REQUIRE(activation == XP_ACT_SILU || activation == XP_ACT_GELU, "%s: unknown activation %d", what, activation);
  XP_REQUIRE(num_experts >= 1 && num_experts <= INT32_MAX, "%s: %lld experts", what, (long long)num_experts);
  XP_REQUIRE(H > 0 && I > 0 && H % kBN == 0 && I % kBN == 0, "%s: H=%lld and I=%lld must be multiples of %d", what,
             (long long)H, (long long)I, kBN);
  XP_REQUIRE(slots >= 1 && slots <= kMaxRouteSlots, "%s: %lld slots (at most %d)", what, (long long)slots,
             kMaxRouteSlots);
  XP_REQUIRE(x && topk_ids && expert_map && topk_weight && w13 && w13_scale && w2 && w2_scale && out,
             "%s: null argument", what);
  XP_REQUIRE(aligned16(x) && aligned16(w13) && aligned16(w2) && aligned16(out), "%s: misaligned buffer", what);
  XP_REQUIRE(work && (reinterpret_cast<uintptr_t>(work) & 255) == 0,
             "%s: the workspace must be non-null and 256-byte aligned", what);
  const int64_t need = xp_moe_workspace_bytes(npairs, I);
  XP_REQUIRE(work_bytes >= need, "%s: workspace of %lld B, needs %lld", what, (long long)work_bytes, (long long)need);
  Work w;
  work_layout(npairs, I, &w, static_cast<uint8_t*>(work));
  // One workgroup per 16-row subtile of an occupied slot and 16 columns.
  // The subtiles number at most min(npairs, slots), plus npairs / 16 when a
  // slot can hold more than 16 pairs (sum over slots of ceil(c / 16) with
  // the counts c summing to npairs).
  const int64_t subs = (npairs < slots ? npairs : slots) + (npairs > 16 ? npairs / 16 : 0);
  const int64_t subs8 = (subs + 7) / 8 * 8;  // the XCD-aware grid covers whole groups of 8
  const dim3 g1(static_cast<unsigned>(subs8 * (I / 16)));
  if (activation == XP_ACT_GELU)
    hipLaunchKernelGGL(gemm1_decode_kernel<XP_ACT_GELU>, g1, dim3(kThreads), static_cast<size_t>(16 * H),
                       as_stream(stream), x, H, I, topk_ids, topk_elem_bytes, static_cast<int>(npairs),
                       static_cast<int>(topk), expert_map, pair_slot, static_cast<int>(num_experts),
                       static_cast<int>(slots), w13, w13_scale, w);
  else
    hipLaunchKernelGGL(gemm1_decode_kernel<XP_ACT_SILU>, g1, dim3(kThreads), static_cast<size_t>(16 * H),
                       as_stream(stream), x, H, I, topk_ids, topk_elem_bytes, static_cast<int>(npairs),
                       static_cast<int>(topk), expert_map, pair_slot, static_cast<int>(num_experts),
                       static_cast<int>(slots), w13, w13_scale, w);
  int rc = check_launch("gemm1_decode_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(gemm2_decode_kernel, dim3(static_cast<unsigned>(T * (H / kDecodeCols2))), dim3(kThreads),
                     static_cast<size_t>(topk * I), as_stream(stream), H, I, static_cast<int>(topk), topk_weight,
                     w2, w2_scale, w, out);
  return check_launch("gemm2_decode_kernel");
}

int xp_moe_topk_sum(const uint16_t* contrib, int64_t T, int64_t topk, int64_t H, const void* topk_ids,
                    int topk_elem_bytes, int64_t num_experts, uint16_t* out, void* stream) {
  XP_REQUIRE(T >= 0 && T <= 65535 && topk >= 1 && H > 0 && H % 8 == 0,
             "xp_moe_topk_sum: T=%lld (at most 65535), topk=%lld, H=%lld (a multiple of 8)", (long long)T,
             (long long)topk, (long long)H);
  XP_REQUIRE(topk_elem_bytes == 4 || topk_elem_bytes == 8, "xp_moe_topk_sum: id size %d", topk_elem_bytes);
  if (T == 0) return XP_OK;
  XP_REQUIRE(contrib && out && topk_ids && aligned16(contrib) && aligned16(out),
             "xp_moe_topk_sum: null or misaligned buffer");
  const unsigned bx = static_cast<unsigned>((H / 8 + 255) / 256);
  if (topk_elem_bytes == 8)
    hipLaunchKernelGGL(topk_sum_kernel<int64_t>, dim3(bx, static_cast<unsigned>(T)), dim3(256), 0, as_stream(stream),
                       contrib, H, static_cast<int>(topk), static_cast<const int64_t*>(topk_ids),
                       static_cast<int>(num_experts), out);
  else
    hipLaunchKernelGGL(topk_sum_kernel<int32_t>, dim3(bx, static_cast<unsigned>(T)), dim3(256), 0, as_stream(stream),
                       contrib, H, static_cast<int>(topk), static_cast<const int32_t*>(topk_ids),
                       static_cast<int>(num_experts), out);
  return check_launch("topk_sum_kernel");
}

}  // extern "C"
