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
// a = bf16(silu(gate) * up); a -> fp8 per 128-group; y likewise with w2;
// contribution = bf16(y * routed weight).
//
// Work decomposition: route lists the pairs of each slab slot in CSR form
// and cuts them into tiles of 64 pairs of one slot. gemm1 takes one tile
// and 128 activation columns per workgroup at prefill sizes; for few pairs
// it takes 16 rows and 16 columns, with the K blocks split over its waves
// (so a decode step of 8 pairs spreads over 256 workgroups). gemm2 takes
// one tile (or 16 rows) and 128 output columns. Launch grids
// are sized from the shapes alone (a bound on the tile count), so the
// sequence is graph-capturable; workgroups past the live tile count exit at
// once.
#include <hip/hip_bf16.h>

#include <mutex>

#include "common.h"

namespace xp {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 64;          // pairs per tile
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
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 16));
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

// Exclusive scan of two counters over a 1024-thread workgroup.
__device__ __forceinline__ int2 block_scan2(int a, int b, int2* s_tot, int2* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int ia = a, ib = b;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int ya = __shfl_up(ia, off, 64), yb = __shfl_up(ib, off, 64);
    if (lane >= off) {
      ia += ya;
      ib += yb;
    }
  }
  if (lane == 63) s_tot[wave] = make_int2(ia, ib);
  __syncthreads();
  int2 base = make_int2(0, 0), all = make_int2(0, 0);
  for (int w = 0; w < kRouteThreads / 64; ++w) {
    const int2 v = s_tot[w];
    if (w < wave) {
      base.x += v.x;
      base.y += v.y;
    }
    all.x += v.x;
    all.y += v.y;
  }
  *total = all;
  return make_int2(base.x + ia - a, base.y + ib - b);
}

// ---- routing: CSR lists of the pairs of each slab slot, and the tiles ----
// offsets[slots + 1]; pairs[offsets[s] .. offsets[s+1]) = pair ids t*topk + k
// of slot s; tiles[0] = live tile count, then (slot, first pair position)
// per tile. Each wave counts a contiguous range of pairs into its own LDS
// histogram (no contention between waves), so a slot's list is ordered by
// wave range; dynamic LDS = 16 * slots ints.
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
                                            int32_t* __restrict__ tiles, int* s_hist, int2* s_tot) {
  constexpr int kW = kRouteThreads / 64;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int i = tid; i < kW * slots; i += kRouteThreads) s_hist[i] = 0;
  __syncthreads();
  const int64_t per = (npairs + kW - 1) / kW;
  const int64_t lo = wave * per, hi = lo + per < npairs ? lo + per : npairs;
  int* hist = s_hist + wave * slots;
  for (int64_t b = lo; b < hi; b += 64 * kRouteBatch) {
    int sl[kRouteBatch];
    route_slots(ids, eb, b + lane, hi, expert_map, E, slots, sl);
#pragma unroll
    for (int j = 0; j < kRouteBatch; ++j)
      if (sl[j] >= 0) atomicAdd(&hist[sl[j]], 1);
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
  const int nt = (c + kBM - 1) / kBM;
  int2 total;
  const int2 off = block_scan2(c, nt, s_tot, &total);
  if (tid < slots) {
    offsets[tid] = off.x;
    for (int w = 0; w < kW; ++w) s_hist[w * slots + tid] += off.x;  // scatter cursors
    for (int i = 0; i < nt; ++i) {
      tiles[1 + 2 * (off.y + i)] = tid;
      tiles[2 + 2 * (off.y + i)] = off.x + i * kBM;
    }
  }
  if (tid == 0) {
    offsets[slots] = total.x;
    tiles[0] = total.y;
  }
  __syncthreads();
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
                                                              int32_t* __restrict__ tiles) {
  extern __shared__ int s_hist[];  // [16 waves][slots]
  __shared__ int2 s_tot[kRouteThreads / 64];
  route_block(ids, eb, npairs, expert_map, E, slots, offsets, pairs, tiles, s_hist, s_tot);
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
                                                                    int32_t* __restrict__ tiles) {
  extern __shared__ int s_hist[];
  __shared__ int2 s_tot[kRouteThreads / 64];
  if (blockIdx.x == 0) {
    route_block(ids, eb, npairs, expert_map, E, slots, offsets, pairs, tiles, s_hist, s_tot);
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

// Tile rows: the pair of each row (-1 for padding) and the A row it reads
// (padding rows repeat the tile's first pair, so every load stays inside
// the operand).
__device__ __forceinline__ void tile_rows(const Tile& tile, const int32_t* pairs, int div, int* s_pair, int* s_row) {
  const int tid = threadIdx.x;
  if (tid < kBM) {
    const int p = pairs[tile.first + (tid < tile.count ? tid : 0)];
    s_pair[tid] = tid < tile.count ? p : -1;
    s_row[tid] = p / div;
  }
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
constexpr int kWideNW = 8;      // waves (16 activation columns each) of a wide gemm1 workgroup
constexpr int kNarrowChunk = 4; // K blocks per load chunk of the small-batch GEMMs
constexpr int kMaxKB = 64;    // K blocks a workgroup keeps row scales for (H, I <= 8192)

constexpr int kAPitch = 144;  // LDS bytes per staged A row (128 + 16 against bank conflicts)

// The A rows of a tile for one K block, staged through registers into LDS
// by all NT threads of the workgroup (16 bytes per thread per piece), so
// the global loads of the next block are in flight while this one is used.
template <int NT>
struct AStage {
  static constexpr int kPer = kBM * 8 / NT;  // 16-byte pieces per thread
  const uint8_t* src[kPer];
  int dst[kPer];
  u32x4 v[kPer];
  __device__ __forceinline__ void init(const uint8_t* A, int64_t lda, const int* s_row) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = static_cast<int>(threadIdx.x) + NT * i, row = c >> 3, off = (c & 7) * 16;
      src[i] = A + static_cast<int64_t>(s_row[row]) * lda + off;
      dst[i] = row * kAPitch + off;
    }
  }
  __device__ __forceinline__ void load(int kb) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = *reinterpret_cast<const u32x4*>(src[i] + kb * kKB);
  }
  __device__ __forceinline__ void store(uint8_t* s_a) const {
#pragma unroll
    for (int i = 0; i < kPer; ++i) *reinterpret_cast<u32x4*>(s_a + dst[i]) = v[i];
  }
};

__device__ __forceinline__ void read_a(const uint8_t* s_a, int row, int q, u32x4 (&a)[2]) {
  const u32x4* p = reinterpret_cast<const u32x4*>(s_a + row * kAPitch + 32 * q);
  a[0] = p[0];
  a[1] = p[1];
}

// GEMM1: gate and up for NW*16 = 128 activation columns of one tile (1-D
// grid in XCD order, see xcd_item); each wave owns 16 columns and runs the K
// blocks in order, so a column's value does not depend on the workgroup
// width. The tile's A rows are staged in LDS, double-buffered, one block
// ahead. Then a = bf16(silu(bf16 gate) * bf16 up) is quantised to fp8 per
// row over the workgroup's 128 columns, one scale group. Only the 16-row
// subtiles that hold pairs are multiplied.
template <int NW>
__global__ void __launch_bounds__(NW * 64) gemm1_kernel(const uint8_t* __restrict__ xq, const float* __restrict__ xs,
                                                        int64_t H, int64_t I, int topk,
                                                        const uint8_t* __restrict__ w13,
                                                        const float* __restrict__ w13_scale,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ pairs,
                                                        const int32_t* __restrict__ tiles, Work work) {
  constexpr int NT = NW * 64, NC = NW * 16;
  __shared__ int s_row[kBM];
  __shared__ int s_pair[kBM];
  __shared__ float s_xs[kBM * kMaxKB];  // token scales per row and K block
  __shared__ float s_sw[2][kMaxKB];     // gate and up weight scales per K block
  __shared__ float s_m[NW][kBM];        // row maxima per wave (16 columns)
  __shared__ __attribute__((aligned(16))) uint8_t s_a[2][kBM * kAPitch];  // A stages; then the bf16 staging

  Tile tile;
  int ti, cb;
  xcd_item(static_cast<int>(I / NC), ti, cb);
  if (!load_tile_at(ti, tiles, offsets, tile)) return;
  const int c0 = cb * NC;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(H / kKB);
  const int nmi = (tile.count + 15) >> 4;

  tile_rows(tile, pairs, topk, s_pair, s_row);
  __syncthreads();
  for (int i = tid; i < 16 * nmi * KB; i += NT) {
    const int r = i / KB, kb = i - r * KB;
    s_xs[i] = xs[static_cast<int64_t>(s_row[r]) * KB + kb];
  }
  {
    // The workgroup's gate and up rows each lie in one 128-row scale block.
    const float* sg = w13_scale + (static_cast<int64_t>(tile.slot) * (2 * I / kKB) + c0 / kKB) * KB;
    const float* su = w13_scale + (static_cast<int64_t>(tile.slot) * (2 * I / kKB) + (I + c0) / kKB) * KB;
    for (int i = tid; i < 2 * KB; i += NT) s_sw[i / KB][i % KB] = (i < KB ? sg : su)[i % KB];
  }
  AStage<NT> st0, st1;  // token rows of two K blocks in flight
  st0.init(xq, H, s_row);
  st1.init(xq, H, s_row);

  const uint8_t* wslot = w13 + static_cast<int64_t>(tile.slot) * 2 * I * H;
  const int64_t n = c0 + 16 * wave + j;
  const uint8_t* brow[2] = {wslot + n * H + 32 * q, wslot + (I + n) * H + 32 * q};

  f32x4 acc[4][2];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 b0[2][2], b1[2][2];
  auto load_b = [&](u32x4 (&b)[2][2], int kb) {
#pragma unroll
    for (int si = 0; si < 2; ++si) load32(brow[si] + kb * kKB, b[si]);
  };
  auto compute = [&](const uint8_t* sa_buf, const u32x4 (&b)[2][2], int kb) {
    const float g = s_sw[0][kb], u = s_sw[1][kb];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      if (mi >= nmi) continue;
      u32x4 a[2];
      read_a(sa_buf, 16 * mi + j, q, a);
      // One combined scale per output row and K block (token scale x weight
      // scale), so each MFMA output needs a single FMA.
      float sc[2][4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sa = s_xs[(16 * mi + 4 * q + r) * KB + kb];
        sc[0][r] = sa * g;
        sc[1][r] = sa * u;
      }
#pragma unroll
      for (int si = 0; si < 2; ++si) {
        const f32x4 part = mfma_k128(a, b[si]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mi][si][r] = fmaf(part[r], sc[si][r], acc[mi][si][r]);
      }
    }
  };

  // Token rows are loaded two K blocks ahead of their multiply and stored to
  // LDS one block ahead; weight rows one block ahead. Block indices are
  // clamped at the last block, so the loads are unconditional.
  auto clampk = [&](int k) { return k < KB ? k : KB - 1; };
  __syncthreads();  // s_row, s_xs, s_sw
  st0.load(0);
  st1.load(clampk(1));
  load_b(b0, 0);
  st0.store(s_a[0]);
  __syncthreads();
  for (int kb = 0; kb < KB; kb += 2) {
    st0.load(clampk(kb + 2));
    load_b(b1, clampk(kb + 1));
    compute(s_a[0], b0, kb);
    st1.store(s_a[1]);
    __syncthreads();
    st1.load(clampk(kb + 3));
    load_b(b0, clampk(kb + 2));
    if (kb + 1 < KB) compute(s_a[1], b1, kb + 1);
    st0.store(s_a[0]);
    __syncthreads();
  }

  static_assert(NC == kKB, "a workgroup covers one 128-column scale group of the activations");
  {
    // 128 columns: one whole scale group of the activations, so they are
    // quantised here (s = max(max |a|, 1e-10) / 448, q = rne(clamp(a / s)),
    // the rule gemm2_narrow_kernel applies, on the same bf16 values).
    float av[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      if (mi >= nmi) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float g = bf16_round(acc[mi][0][r]), u = bf16_round(acc[mi][1][r]);
        const float a = bf16_round(g / (1.0f + expf(-g)) * u);
        av[mi][r] = a;
        float m = fabsf(a);
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 16));
        if (j == 0) s_m[wave][16 * mi + 4 * q + r] = m;
      }
    }
    __syncthreads();
    float* s_q = s_m[0];  // row scales, written over wave 0's maxima after all are read
    float qs = 0.f;
    if (tid < kBM) {
      float m = s_m[0][tid];
#pragma unroll
      for (int w = 1; w < NW; ++w) m = fmaxf(m, s_m[w][tid]);
      qs = quant_scale(m);
    }
    __syncthreads();
    if (tid < kBM) {
      s_q[tid] = qs;
      const int p = s_pair[tid];
      if (p >= 0) work.acts[static_cast<int64_t>(p) * (I / kKB) + c0 / kKB] = qs;
    }
    __syncthreads();
    uint8_t* s_act = s_a[0];  // [kBM][128] fp8
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      if (mi >= nmi) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mi + 4 * q + r;
        s_act[row * kKB + 16 * wave + j] = static_cast<uint8_t>(to_fp8(clamp_fp8(av[mi][r] / s_q[row])));
      }
    }
    __syncthreads();
    for (int i = tid; i < kBM * (kKB / 16); i += NT) {  // 16-byte pieces
      const int row = i / (kKB / 16), piece = i - row * (kKB / 16);
      const int p = s_pair[row];
      if (p >= 0)
        *reinterpret_cast<u32x4*>(work.act + static_cast<int64_t>(p) * I + c0 + piece * 16) =
            *reinterpret_cast<const u32x4*>(s_act + row * kKB + piece * 16);
    }
  }
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
      const float g = bf16_round(acc[0][r]), u = bf16_round(acc[1][r]);
      const float a = bf16_round(g / (1.0f + expf(-g)) * u);
      float m = fabsf(a);
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) m = fmaxf(m, __shfl_xor(m, off, 16));
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
  if (!load_tile_at(ti, tiles, offsets, tile)) return;
  const int sub = item / ncb, r0 = 16 * sub;
  if (r0 >= tile.count) return;
  const int n0 = (item - sub * ncb) * kBN;
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

// GEMM2: down projection of 128 output columns times the routed weight,
// bf16 rows per pair; each wave owns 32 columns and runs the K blocks in
// order over the tile's fp8 activations, staged in LDS one block ahead.
// 1-D grid in XCD order (see xcd_item).
__global__ void __launch_bounds__(kThreads) gemm2_kernel(int64_t H, int64_t I, const float* __restrict__ topk_weight,
                                                         const uint8_t* __restrict__ w2,
                                                         const float* __restrict__ w2_scale,
                                                         const int32_t* __restrict__ offsets,
                                                         const int32_t* __restrict__ pairs,
                                                         const int32_t* __restrict__ tiles, Work work,
                                                         uint16_t* __restrict__ out) {
  __shared__ int s_row[kBM];
  __shared__ int s_pair[kBM];
  __shared__ float s_as[kBM * kMaxKB];
  __shared__ float s_w[kBM];
  __shared__ float s_sw[kMaxKB];  // weight scales per K block of this 128-column block
  __shared__ __attribute__((aligned(16))) uint8_t s_a[2][kBM * kAPitch];
  __shared__ __attribute__((aligned(16))) uint16_t s_o[kBM * kBN];

  Tile tile;
  int ti, cb;
  xcd_item(static_cast<int>(H / kBN), ti, cb);
  if (!load_tile_at(ti, tiles, offsets, tile)) return;
  const int n0 = cb * kBN;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int q = lane >> 4, j = lane & 15;
  const int KB = static_cast<int>(I / kKB);
  const int nmi = (tile.count + 15) >> 4;

  tile_rows(tile, pairs, 1, s_pair, s_row);
  __syncthreads();
  for (int i = tid; i < 16 * nmi * KB; i += kThreads) {
    const int r = i / KB, kb = i - r * KB;
    s_as[i] = work.acts[static_cast<int64_t>(s_row[r]) * KB + kb];
  }
  if (tid < kBM) s_w[tid] = s_pair[tid] >= 0 ? topk_weight[s_pair[tid]] : 0.f;
  if (tid < KB) s_sw[tid] = w2_scale[(static_cast<int64_t>(tile.slot) * (H / kKB) + n0 / kKB) * KB + tid];
  AStage<kThreads> st0, st1;  // activation rows of two K blocks in flight
  st0.init(work.act, I, s_row);
  st1.init(work.act, I, s_row);

  const uint8_t* wslot = w2 + static_cast<int64_t>(tile.slot) * H * I;
  const uint8_t* brow[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) brow[t] = wslot + static_cast<int64_t>(n0 + 32 * wave + 16 * t + j) * I + 32 * q;

  f32x4 acc[4][2];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) acc[mi][0] = acc[mi][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 b0[2][2], b1[2][2];
  auto load_b = [&](u32x4 (&b)[2][2], int kb) {
#pragma unroll
    for (int t = 0; t < 2; ++t) load32(brow[t] + kb * kKB, b[t]);
  };
  auto compute = [&](const uint8_t* sa_buf, const u32x4 (&b)[2][2], int kb) {
    const float w = s_sw[kb];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      if (mi >= nmi) continue;
      u32x4 a[2];
      read_a(sa_buf, 16 * mi + j, q, a);
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = s_as[(16 * mi + 4 * q + r) * KB + kb] * w;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f32x4 part = mfma_k128(a, b[t]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mi][t][r] = fmaf(part[r], sc[r], acc[mi][t][r]);
      }
    }
  };

  // As in gemm1_kernel: activation rows two K blocks ahead, weights one.
  auto clampk = [&](int k) { return k < KB ? k : KB - 1; };
  __syncthreads();  // s_row, s_as, s_w, s_sw
  st0.load(0);
  st1.load(clampk(1));
  load_b(b0, 0);
  st0.store(s_a[0]);
  __syncthreads();
  for (int kb = 0; kb < KB; kb += 2) {
    st0.load(clampk(kb + 2));
    load_b(b1, clampk(kb + 1));
    compute(s_a[0], b0, kb);
    st1.store(s_a[1]);
    __syncthreads();
    st1.load(clampk(kb + 3));
    load_b(b0, clampk(kb + 2));
    if (kb + 1 < KB) compute(s_a[1], b1, kb + 1);
    st0.store(s_a[0]);
    __syncthreads();
  }

#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    if (mi >= nmi) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * mi + 4 * q + r;
      const float wgt = s_w[row];
#pragma unroll
      for (int t = 0; t < 2; ++t)
        s_o[row * kBN + 32 * wave + 16 * t + j] = static_cast<uint16_t>(bf16_bits(acc[mi][t][r] * wgt));
    }
  }
  __syncthreads();
  // 256 bytes per row: 16 threads x 16 bytes, 16 rows per pass.
  for (int row = tid >> 4; row < tile.count; row += kThreads / 16) {
    const int p = s_pair[row];
    const int col = (tid & 15) * 8;
    *reinterpret_cast<u32x4*>(out + static_cast<int64_t>(p) * H + n0 + col) =
        *reinterpret_cast<const u32x4*>(s_o + row * kBN + col);
  }
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
  return (npairs + kBM - 1) / kBM + (slots < npairs ? slots : npairs);
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
  hipLaunchKernelGGL(route_kernel, dim3(1), dim3(kRouteThreads), lds, as_stream(stream), topk_ids, topk_elem_bytes,
                     T * topk, expert_map, static_cast<int>(num_experts), static_cast<int>(slots), offsets, pairs,
                     tiles);
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
  hipLaunchKernelGGL(quant_route_kernel, dim3(grid), dim3(kRouteThreads), lds, as_stream(stream), x, T, H, xq, xs,
                     topk_ids, topk_elem_bytes, T * topk, expert_map, static_cast<int>(num_experts),
                     static_cast<int>(slots), offsets, pairs, tiles);
  return check_launch("quant_route_kernel");
}

int64_t xp_moe_workspace_bytes(int64_t npairs, int64_t I) {
  if (npairs <= 0 || I <= 0) return 0;
  return work_layout(npairs, I, nullptr, nullptr);
}

}  // extern "C"

namespace xp {
namespace {

// Argument checks shared by xp_moe_experts and xp_moe_experts_noalloc (all
// but the workspace's).
int check_experts(const char* what, const uint8_t* xq, const float* xs, int64_t T, int64_t topk,
                  const float* topk_weight, int64_t H, int64_t I, const uint8_t* w13, const float* w13_scale,
                  const uint8_t* w2, const float* w2_scale, int64_t slots, const int32_t* offsets,
                  const int32_t* pairs, const int32_t* tiles, const uint16_t* out) {
  XP_REQUIRE(H > 0 && I > 0 && H % kBN == 0 && I % kBN == 0 && H <= kKB * kMaxKB && I <= kKB * kMaxKB,
             "%s: H=%lld and I=%lld must be multiples of %d, at most %d", what, (long long)H, (long long)I, kBN,
             kKB * kMaxKB);
  XP_REQUIRE(T >= 0 && topk >= 1 && T * topk <= INT32_MAX && slots >= 1 && slots <= kMaxRouteSlots,
             "%s: T=%lld, topk=%lld, slots=%lld", what, (long long)T, (long long)topk, (long long)slots);
  if (T == 0) return XP_OK;
  XP_REQUIRE(xq && xs && topk_weight && w13 && w13_scale && w2 && w2_scale && offsets && pairs && tiles && out,
             "%s: null argument", what);
  XP_REQUIRE(aligned16(xq) && aligned16(w13) && aligned16(w2) && aligned16(out),
             "%s: fp8 and output buffers must be 16-byte aligned", what);
  const int64_t bound = xp_moe_max_tiles(T * topk, slots);
  XP_REQUIRE(bound <= 65535, "%s: %lld tiles exceed the launch grid", what, (long long)bound);
  return XP_OK;
}

// The two (or, for few pairs, narrow) GEMM launches of one expert call over a
// workspace of xp_moe_workspace_bytes(T * topk, I) bytes at `work`.
int launch_experts(const uint8_t* xq, const float* xs, int64_t T, int64_t topk, const float* topk_weight, int64_t H,
                   int64_t I, const uint8_t* w13, const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                   int64_t slots, const int32_t* offsets, const int32_t* pairs, const int32_t* tiles, uint8_t* work,
                   uint16_t* out, void* stream) {
  const int64_t npairs = T * topk;
  const int64_t bound = xp_moe_max_tiles(npairs, slots);
  Work w;
  work_layout(npairs, I, &w, work);
  const int64_t tiles8 = (bound + 7) / 8 * 8;  // the XCD-aware grids cover whole groups of 8 tiles
  const int64_t g2 = tiles8 * (H / kBN);
  XP_REQUIRE(g2 <= INT32_MAX, "xp_moe_experts: grid too large");
  // Prefill-sized calls take 16*kWideNW = 128 activation columns of a tile
  // per workgroup (token rows shared by more waves) and quantise them there;
  // small calls take 16 rows x 16 columns (more workgroups for few pairs)
  // and the small-batch gemm2 quantises. Every column is computed the same
  // way in both.
  const bool narrow = bound < kWideTiles;
  // 16-row subtiles a tile can have: a tile holds at most min(64, npairs) pairs.
  const int nsub = static_cast<int>(((npairs < kBM ? npairs : kBM) + 15) / 16);
  if (!narrow) {
    const int64_t g1w = tiles8 * (I / (16 * kWideNW));
    hipLaunchKernelGGL(gemm1_kernel<kWideNW>, dim3(static_cast<unsigned>(g1w)), dim3(64 * kWideNW), 0,
                       as_stream(stream), xq, xs,
                       H, I, static_cast<int>(topk), w13, w13_scale, offsets, pairs, tiles, w);
  } else {
    // Few pairs: 16-row subtiles x 16 columns, the K blocks split over 4 waves.
    const int64_t g1n = tiles8 * nsub * (I / 16);
    XP_REQUIRE(g1n <= INT32_MAX, "xp_moe_experts: grid too large");
    hipLaunchKernelGGL(gemm1_narrow_kernel, dim3(static_cast<unsigned>(g1n)), dim3(kThreads), 0, as_stream(stream), xq,
                       xs, H, I, static_cast<int>(topk), w13, w13_scale, offsets, pairs, tiles, nsub, w);
  }
  int rc = check_launch("gemm1_kernel");
  if (rc) return rc;
  if (narrow)
    hipLaunchKernelGGL(gemm2_narrow_kernel<kNarrowChunk>, dim3(static_cast<unsigned>(nsub * g2)), dim3(kThreads), 0,
                       as_stream(stream), H, I, topk_weight, w2, w2_scale, offsets, pairs, tiles, nsub, w, out);
  else
    hipLaunchKernelGGL(gemm2_kernel, dim3(static_cast<unsigned>(g2)), dim3(kThreads), 0, as_stream(stream), H, I,
                       topk_weight, w2, w2_scale, offsets, pairs, tiles, w, out);
  return check_launch("gemm2_kernel");
}

}  // namespace
}  // namespace xp

// Workspace of xp_moe_experts_noalloc, one copy on every device the library
// runs on (held until the process ends). Host code never passes this name to
// a kernel: it stands for the host-side shadow, and each device's own
// address comes from hipGetSymbolAddress (scratch_address).
static __device__ __align__(256) uint8_t scratch[XP_MOE_SCRATCH_BYTES];

namespace xp {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices];  // device address of `scratch`, per device

// The current device's address of `scratch`, looked up on the first call on
// that device (with it current) and kept.
int scratch_address(uint8_t** out) {
  int dev = -1;
  XP_HIP(hipGetDevice(&dev));
  XP_REQUIRE(dev >= 0 && dev < kMaxDevices, "xp_moe_experts_noalloc: device %d (at most %d devices)", dev,
             kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(XP_E_HIP, "xp_moe_experts_noalloc: hipGetSymbolAddress(scratch) on device %d failed: %s", dev,
                  hipGetErrorString(e));
    g_scratch[dev] = static_cast<uint8_t*>(p);
  }
  *out = g_scratch[dev];
  return XP_OK;
}

}  // namespace
}  // namespace xp

extern "C" {

int xp_moe_experts(const uint8_t* xq, const float* xs, int64_t T, int64_t topk, const float* topk_weight, int64_t H,
                   int64_t I, const uint8_t* w13, const float* w13_scale, const uint8_t* w2, const float* w2_scale,
                   int64_t slots, const int32_t* offsets, const int32_t* pairs, const int32_t* tiles, void* work,
                   int64_t work_bytes, uint16_t* out, void* stream) {
  int rc = check_experts("xp_moe_experts", xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2, w2_scale, slots,
                         offsets, pairs, tiles, out);
  if (rc || T == 0) return rc;
  XP_REQUIRE(work && (reinterpret_cast<uintptr_t>(work) & 255) == 0,
             "xp_moe_experts: the workspace must be non-null and 256-byte aligned");
  const int64_t need = xp_moe_workspace_bytes(T * topk, I);
  XP_REQUIRE(work_bytes >= need, "xp_moe_experts: workspace of %lld B, needs %lld", (long long)work_bytes,
             (long long)need);
  return launch_experts(xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2, w2_scale, slots, offsets, pairs,
                        tiles, static_cast<uint8_t*>(work), out, stream);
}

int xp_moe_experts_noalloc(const uint8_t* xq, const float* xs, int64_t T, int64_t topk, const float* topk_weight,
                           int64_t H, int64_t I, const uint8_t* w13, const float* w13_scale, const uint8_t* w2,
                           const float* w2_scale, int64_t slots, const int32_t* offsets, const int32_t* pairs,
                           const int32_t* tiles, uint16_t* out, void* stream) {
  int rc = check_experts("xp_moe_experts_noalloc", xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2,
                         w2_scale, slots, offsets, pairs, tiles, out);
  if (rc || T == 0) return rc;
  const int64_t need = xp_moe_workspace_bytes(T * topk, I);
  if (need > XP_MOE_SCRATCH_BYTES)
    return fail(XP_E_LIMIT,
                "xp_moe_experts_noalloc: %lld pairs x I=%lld need a workspace of %lld B, above the library's "
                "%lld B; call xp_moe_experts with a workspace instead",
                (long long)(T * topk), (long long)I, (long long)need, (long long)XP_MOE_SCRATCH_BYTES);
  uint8_t* work = nullptr;
  rc = scratch_address(&work);
  if (rc) return rc;
  return launch_experts(xq, xs, T, topk, topk_weight, H, I, w13, w13_scale, w2, w2_scale, slots, offsets, pairs,
                        tiles, work, out, stream);
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
