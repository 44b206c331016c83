// Batched GPU encoder of the fp8 exponent Huffman row format
// (encode, codec.py:125-198), producing the bytes of the host encoder
// (codec_host.cpp) and of the reference. Two launches:
//
// encode_plan_kernel, one workgroup per row:
//   1. exponent histogram: per-thread counters in LDS, then summed;
//   2. the code (code_build.h) by one thread, the 512-entry LUT by all;
//   3. Huffman words per chunk: the decoder loads a word before symbol i
//      whenever fewer than LIMIT bits are left, so a chunk whose last symbol
//      starts at bit b needs (b + LIMIT - 1) / 32 + 1 words; summed per
//      group and scanned into gstart, written to the record's header.
// encode_groups_kernel, one workgroup per 8 groups of a row:
//   4. the code again, from the row's LUT (every symbol has a code of at
//      most LIMIT bits, so each one appears in the 9-bit table with its
//      length, and the canonical codes follow from the lengths); then each
//      32-lane half-wave encodes one group: its lanes walk their chunks
//      in lockstep, run the decoder's refill rule, and give each word the
//      (symbol index, lane) rank of its refill -- the wave ballot's count of
//      refilling lanes below, as the decoder computes it. A lane emits a
//      word once its 32 bits are complete; at most two refills are waiting
//      for their word. The lane also writes its sign/mantissa nibble words.
// The record is written whole: gstart and the zero tail up to the pitch by
// the first launch, nibbles and Huffman words by the second. A row that does
// not fit its pitch writes nothing but its LUT and needed bytes.
#include "code_build.h"
#include "common.h"

namespace xp {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxGroups = 4096;  // groups per row a workgroup scans in LDS
constexpr int kGroupsPerBlock = 2 * kThreads / 64;  // 8: one per half-wave
// The plan's two passes over a row run in one workgroup per row: 16 waves,
// each lane with four 16-byte loads in flight, so that a pass is not a
// chain of load latencies.
constexpr int kPlanThreads = 1024;
constexpr int kPlanUnroll = 4;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct EncodeArgs {
  const uint8_t* raw;
  int64_t raw_stride;  // bytes between rows of raw
  int64_t n;           // values per row
  int chunk;           // values per lane chunk (a power of two, 16..1024)
  int G;               // groups per row
  uint8_t* rec;
  int64_t pitch;       // bytes between records, the record size
  uint8_t* lut;
  int64_t lut_stride;  // bytes between LUTs
  int64_t* needed;     // record bytes each row needs
};

// Lengths of the four bytes of w as a sum. lb[k] holds the code lengths of
// symbols 4k..4k+3 as bytes. Each byte's symbol (its exponent field) selects
// its length with byte permutes: one over symbols 0-7, one over 8-15, and a
// third that takes each byte from the one its symbol's bit 3 names; a sum
// of absolute byte differences against zero adds the four lengths.
__device__ __forceinline__ uint32_t sum_lengths4(uint32_t w, const uint32_t (&lb)[4]) {
  const uint32_t sym = (w >> 3) & 0x0f0f0f0fu;
  const uint32_t low = sym & 0x07070707u;
  const uint32_t a = __builtin_amdgcn_perm(lb[1], lb[0], low);  // symbols 0-7
  const uint32_t b = __builtin_amdgcn_perm(lb[3], lb[2], low);  // symbols 8-15
  const uint32_t pick = ((sym >> 1) & 0x04040404u) | 0x03020100u;  // byte i of a, or of b for symbols 8-15
  return __builtin_amdgcn_sad_u8(__builtin_amdgcn_perm(b, a, pick), 0u, 0u);
}

__global__ void __launch_bounds__(kPlanThreads) encode_plan_kernel(EncodeArgs a) {
  __shared__ uint32_t s_hist[code::kSyms][kPlanThreads];  // per-thread counters
  __shared__ int32_t s_len[code::kSyms];
  __shared__ int32_t s_code[code::kSyms];
  __shared__ int32_t s_words[kMaxGroups + 1];          // words per group, then gstart
  __shared__ int64_t s_total;

  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint8_t* raw = a.raw + static_cast<int64_t>(row) * a.raw_stride;
  uint8_t* rec = a.rec + static_cast<int64_t>(row) * a.pitch;
  const int64_t n = a.n;
  const int chunk = a.chunk, G = a.G;

  // 1. Histogram of the exponent fields. Each thread counts into its own
  // LDS counters with atomic adds whose result is not returned: a plain
  // increment is a read and a write that the next increment of the same
  // counter must wait for, a chain of LDS round trips per byte.
  for (int s = 0; s < code::kSyms; ++s) s_hist[s][tid] = 0;
  constexpr int64_t kStep = int64_t(kPlanThreads) * 16;
  for (int64_t off0 = int64_t(tid) * 16; off0 < n; off0 += kStep * kPlanUnroll) {
    u32x4 v[kPlanUnroll];
#pragma unroll
    for (int u = 0; u < kPlanUnroll; ++u)
      if (off0 + u * kStep < n) v[u] = *reinterpret_cast<const u32x4*>(raw + off0 + u * kStep);
#pragma unroll
    for (int u = 0; u < kPlanUnroll; ++u) {
      if (off0 + u * kStep >= n) continue;
      const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int b = 0; b < 4; ++b) atomicAdd(&s_hist[(w[k] >> (8 * b + 3)) & 15u][tid], 1u);
    }
  }
  __syncthreads();

  // 2. The code, and the LUT. Wave w sums symbol w's counters.
  static_assert(kPlanThreads / 64 == code::kSyms, "one wave per symbol");
  {
    const int sym = tid >> 6, part = tid & 63;
    uint32_t t = 0;
    for (int i = 0; i < kPlanThreads / 64; ++i) t += s_hist[sym][part * (kPlanThreads / 64) + i];
    for (int d = 32; d >= 1; d >>= 1) t += __shfl_xor(t, d, 64);
    if (part == 0) s_hist[sym][0] = t;
  }
  __syncthreads();
  if (tid == 0) {
    int64_t hist[code::kSyms];
    for (int s = 0; s < code::kSyms; ++s) hist[s] = s_hist[s][0];
    int32_t lengths[code::kSyms], codes[code::kSyms];
    code::code_lengths(hist, lengths);
    code::canonical_codes(lengths, codes);
    for (int s = 0; s < code::kSyms; ++s) {
      s_len[s] = lengths[s];
      s_code[s] = codes[s];
    }
  }
  __syncthreads();
  {
    int32_t lengths[code::kSyms], codes[code::kSyms];
    for (int s = 0; s < code::kSyms; ++s) {
      lengths[s] = s_len[s];
      codes[s] = s_code[s];
    }
    uint8_t* lut = a.lut + static_cast<int64_t>(row) * a.lut_stride;
    for (int x = tid; x < XP_LUT_BYTES; x += kPlanThreads)
      lut[x] = static_cast<uint8_t>(code::lut_entry(lengths, codes, x));
  }
  uint32_t lb[4] = {0u, 0u, 0u, 0u};  // the lengths as bytes, symbol s in byte s % 4 of lb[s / 4]
#pragma unroll
  for (int s = 0; s < code::kSyms; ++s) lb[s / 4] |= static_cast<uint32_t>(s_len[s]) << (8 * (s % 4));

  // 3. Words per chunk: (start bit of its last symbol + LIMIT - 1) / 32 + 1.
  // The chunk's 16-byte pieces are spread over consecutive threads, so each
  // chunk is summed by a power-of-two set of lanes of one wave.
  const int per = chunk / 16;  // threads per chunk
  for (int g = tid; g < G; g += kPlanThreads) s_words[g] = 0;
  __syncthreads();
  // A chunk's pieces are all below n or all at or past it (n is a multiple
  // of the chunk), so each set of lanes shuffles together.
  for (int64_t off0 = int64_t(tid) * 16; off0 < n; off0 += kStep * kPlanUnroll) {
    u32x4 v[kPlanUnroll];
#pragma unroll
    for (int u = 0; u < kPlanUnroll; ++u)
      if (off0 + u * kStep < n) v[u] = *reinterpret_cast<const u32x4*>(raw + off0 + u * kStep);
#pragma unroll
    for (int u = 0; u < kPlanUnroll; ++u) {
      const int64_t off = off0 + u * kStep;
      if (off >= n) continue;
      uint32_t bits = sum_lengths4(v[u].x, lb) + sum_lengths4(v[u].y, lb) + sum_lengths4(v[u].z, lb) +
                      sum_lengths4(v[u].w, lb);
      const bool last = ((off + 16) % chunk) == 0;
      if (last) {  // not the last symbol
        const uint32_t s3 = v[u].w >> 27 & 15u;
        const bool hi = s3 >= 8u;
        bits -= __builtin_amdgcn_perm(hi ? lb[3] : lb[1], hi ? lb[2] : lb[0], (s3 & 7u) | 0x0c0c0c00u);
      }
      for (int d = 1; d < per; d <<= 1) bits += __shfl_xor(bits, d, per);
      if (last)
        atomicAdd(&s_words[off / (int64_t(chunk) * XP_LANES)], static_cast<int32_t>((bits + XP_LIMIT - 1) / 32 + 1));
    }
  }
  __syncthreads();
  if (tid == 0) {  // exclusive scan into gstart
    int64_t t = 0;
    for (int g = 0; g < G; ++g) {
      const int32_t w = s_words[g];
      s_words[g] = static_cast<int32_t>(t);
      t += w;
    }
    s_words[G] = static_cast<int32_t>(t);
    s_total = t;
  }
  __syncthreads();
  const int64_t head = 4 * (int64_t(G) + 1) + n / 2;
  const int64_t nbytes = head + 4 * s_total;
  if (tid == 0) a.needed[row] = nbytes;
  if (nbytes > a.pitch) return;

  int32_t* gstart = reinterpret_cast<int32_t*>(rec);
  for (int g = tid; g <= G; g += kPlanThreads) gstart[g] = s_words[g];
  // Zero tail (nbytes and the pitch are multiples of 4).
  for (int64_t i = nbytes / 4 + tid; i < a.pitch / 4; i += kPlanThreads) reinterpret_cast<uint32_t*>(rec)[i] = 0;
}

__global__ void __launch_bounds__(kThreads) encode_groups_kernel(EncodeArgs a, int blocks_per_row) {
  __shared__ int32_t s_len[code::kSyms];
  __shared__ uint32_t s_tab[code::kSyms];  // code | length << 16

  const int row = blockIdx.x / blocks_per_row, part = blockIdx.x % blocks_per_row;
  const int tid = threadIdx.x;
  if (a.needed[row] > a.pitch) return;  // the row does not fit: the plan wrote nothing either
  const uint8_t* raw = a.raw + static_cast<int64_t>(row) * a.raw_stride;
  uint8_t* rec = a.rec + static_cast<int64_t>(row) * a.pitch;
  const int64_t n = a.n;
  const int chunk = a.chunk, G = a.G;
  const int32_t* gstart = reinterpret_cast<const int32_t*>(rec);

  // 4. The code from the LUT (entry = symbol << 4 | length), then groups,
  // one per half-wave.
  const uint8_t* lut = a.lut + static_cast<int64_t>(row) * a.lut_stride;
  for (int x = tid; x < XP_LUT_BYTES; x += kThreads) {
    const uint32_t ent = lut[x];
    s_len[ent >> 4] = static_cast<int32_t>(ent & 15u);  // every entry of a symbol holds the same length
  }
  __syncthreads();
  if (tid == 0) {
    int32_t lengths[code::kSyms], codes[code::kSyms];
    for (int s = 0; s < code::kSyms; ++s) lengths[s] = s_len[s];
    code::canonical_codes(lengths, codes);
    for (int s = 0; s < code::kSyms; ++s)
      s_tab[s] = static_cast<uint32_t>(codes[s]) | (static_cast<uint32_t>(lengths[s]) << 16);
  }
  __syncthreads();

  const int64_t head = 4 * (int64_t(G) + 1) + n / 2;
  uint32_t* fixed = reinterpret_cast<uint32_t*>(rec + 4 * (int64_t(G) + 1));
  uint32_t* huff = reinterpret_cast<uint32_t*>(rec + head);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const bool upper = lane >= 32;
  const uint32_t li = lane & 31;
  const uint32_t half_shift = upper ? 16u : 0u;
  const int mwords = chunk / 8;
  const uint32_t total = static_cast<uint32_t>(gstart[G]);  // every word position is below it
  {
    const int g0 = part * kGroupsPerBlock + 2 * wave;
    if (g0 >= G) return;
    const int g = g0 + (upper ? 1 : 0);
    const bool live = g < G;  // a spare half-wave walks the last group and writes nothing
    const int gg = live ? g : G - 1;
    const uint8_t* src = raw + (int64_t(gg) * XP_LANES + li) * chunk;
    uint32_t* fx = fixed + int64_t(gg) * mwords * XP_LANES + li;
    // Word positions within each half's group, both below 2^16 (a group's
    // words are at most 32 chunks of 9-bit codes), packed in one scalar
    // register: the lower half's in bits 0-15, the upper half's in 16-31
    // biased by kBias, so that lowering the upper half's count by the lower
    // half's refills of a symbol (at most 32) never borrows. A lane's
    // queued positions are relative; gbase makes them absolute.
    constexpr uint32_t kBias = 64;
    const uint32_t gs_lo = static_cast<uint32_t>(gstart[g0]);
    const uint32_t gs_hi = static_cast<uint32_t>(gstart[g0 + 1 < G ? g0 + 1 : G - 1]);
    const uint32_t gbase = upper ? gs_hi - kBias : gs_lo;
    uint32_t offs = kBias << 16;
    uint32_t level = 0;         // bits the decoder has buffered
    uint64_t acc = 0;           // bits of the lane's stream not yet emitted
    uint32_t accbits = 0;
    uint32_t q0 = 0, q1 = 0;    // positions of words refilled but not yet emitted
    uint32_t qn = 0;
    // A lane's values in blocks of 64 (four 16-byte loads back to back, so
    // each cache line of its chunk is fetched about twice instead of once
    // per 16 values), the next block loaded while this one is encoded.
    const int nv = chunk < 64 ? chunk / 16 : 4;  // loads per block
    u32x4 cur[4], nxt[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (j < nv) cur[j] = *reinterpret_cast<const u32x4*>(src + 16 * j);
    const uint8_t* tab = reinterpret_cast<const uint8_t*>(s_tab);
    for (int i0 = 0; i0 < chunk; i0 += 16 * nv) {
      if (i0 + 16 * nv < chunk) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (j < nv) nxt[j] = *reinterpret_cast<const u32x4*>(src + i0 + 16 * nv + 16 * j);
      }
#pragma unroll
      for (int jv = 0; jv < 4; ++jv) {
        if (jv >= nv) break;
        const u32x4 v = cur[jv];
        const int i1 = i0 + 16 * jv;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          // Each byte's exponent field (bits 3-6) as a byte offset into s_tab.
          const uint32_t ex4 = (w[k] >> 1) & 0x3C3C3C3Cu;
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            // The decoder's refill rule: a lane with fewer than LIMIT bits
            // buffered takes the next word of its group, ranked by the
            // refilling lanes below it in its half.
            const bool refill = level < static_cast<uint32_t>(XP_LIMIT);
            const unsigned long long mask = __builtin_amdgcn_ballot_w64(refill);
            const uint32_t m_lo = static_cast<uint32_t>(mask), m_hi = static_cast<uint32_t>(mask >> 32);
            const uint32_t n_lo = static_cast<uint32_t>(__popc(m_lo)), n_hi = static_cast<uint32_t>(__popc(m_hi));
            const uint32_t bases = offs - (n_lo << 16);
            const uint32_t pos = __builtin_amdgcn_mbcnt_hi(
                m_hi, __builtin_amdgcn_mbcnt_lo(m_lo, __builtin_amdgcn_ubfe(bases, half_shift, 16u)));
            offs += n_lo + (n_hi << 16);
            q0 = refill && qn == 0 ? pos : q0;
            q1 = refill && qn != 0 ? pos : q1;
            qn += refill ? 1u : 0u;
            level += refill ? 32u : 0u;
            const uint32_t t = *reinterpret_cast<const uint32_t*>(tab + __builtin_amdgcn_ubfe(ex4, 8u * b, 8u));
            const uint32_t len = t >> 16;
            acc |= static_cast<uint64_t>(t & 0xffffu) << accbits;
            accbits += len;
            level -= len;
            const bool full = accbits >= 32;  // word q0 is complete
            if (full && live && gbase + q0 < total) huff[gbase + q0] = static_cast<uint32_t>(acc);
            acc = full ? acc >> 32 : acc;
            accbits &= 31u;  // below 32 + LIMIT
            q0 = full ? q1 : q0;
            qn -= full ? 1u : 0u;
          }
          if (k & 1) {  // 8 values: one nibble word, value j in bits 4j..4j+3
            // Per byte, sign (bit 7) to bit 3 beside the mantissa (bits 0-2);
            // then two bytes' nibbles joined and the four pairs picked.
            const uint32_t x0 = w[k - 1], x1 = w[k];
            const uint32_t t0 = (x0 & 0x07070707u) | ((x0 >> 4) & 0x08080808u);
            const uint32_t t1 = (x1 & 0x07070707u) | ((x1 >> 4) & 0x08080808u);
            const uint32_t nib = __builtin_amdgcn_perm(t1 | (t1 >> 4), t0 | (t0 >> 4), 0x06040200u);
            if (live) fx[int64_t((i1 + 8 * (k >> 1)) / 8) * XP_LANES] = nib;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) cur[j] = nxt[j];
    }
    // Words whose refill came but whose bits ran out: the rest of the stream,
    // then zeros.
    while (__builtin_amdgcn_ballot_w64(qn > 0)) {
      if (qn > 0) {
        if (live && gbase + q0 < total) huff[gbase + q0] = static_cast<uint32_t>(acc);
        acc >>= 32;
        q0 = q1;
        --qn;
      }
    }
  }
}

}  // namespace
}  // namespace xp

using namespace xp;

extern "C" {

int xp_encode_rows(const uint8_t* raw, int64_t rows, int64_t raw_stride, int64_t n, int64_t chunk, uint8_t* records,
                   int64_t pitch, uint8_t* luts, int64_t lut_stride, int64_t* needed, void* stream) {
  XP_REQUIRE(rows >= 0 && rows <= INT32_MAX, "xp_encode_rows: rows=%lld", (long long)rows);
  if (rows == 0) return XP_OK;
  XP_REQUIRE(raw && records && luts && needed, "xp_encode_rows: null argument");
  XP_REQUIRE(chunk >= 16 && chunk <= 1024 && (chunk & (chunk - 1)) == 0,
             "xp_encode_rows: chunk=%lld (a power of two, 16..1024)", (long long)chunk);
  const int64_t group = chunk * XP_LANES;
  if (n <= 0 || n % group)
    return fail(XP_E_SHAPE, "row of %lld values is not a multiple of %lld", (long long)n, (long long)group);
  const int64_t G = n / group;
  XP_REQUIRE(G <= kMaxGroups, "xp_encode_rows: %lld groups per row (at most %d)", (long long)G, kMaxGroups);
  XP_REQUIRE(raw_stride >= n && raw_stride % 16 == 0 && aligned16(raw),
             "xp_encode_rows: raw rows must be 16-byte aligned with a stride of at least n");
  // A pitch below the header is a row that does not fit (needed > pitch), as
  // in xp_encode_row, not an argument error.
  XP_REQUIRE(pitch > 0 && pitch % 16 == 0 && aligned16(records),
             "xp_encode_rows: pitch %lld is not a positive multiple of 16", (long long)pitch);
  XP_REQUIRE(lut_stride >= XP_LUT_BYTES, "xp_encode_rows: lut_stride=%lld", (long long)lut_stride);
  EncodeArgs a{raw, raw_stride, n, static_cast<int>(chunk), static_cast<int>(G), records, pitch,
               luts, lut_stride, needed};
  const int64_t blocks = (G + kGroupsPerBlock - 1) / kGroupsPerBlock;
  XP_REQUIRE(rows * blocks <= INT32_MAX, "xp_encode_rows: %lld rows x %lld blocks", (long long)rows, (long long)blocks);
  hipLaunchKernelGGL(encode_plan_kernel, dim3(static_cast<unsigned>(rows)), dim3(kPlanThreads), 0, as_stream(stream),
                     a);
  if (int rc = check_launch("encode_plan_kernel")) return rc;
  hipLaunchKernelGGL(encode_groups_kernel, dim3(static_cast<unsigned>(rows * blocks)), dim3(kThreads), 0,
                     as_stream(stream), a, static_cast<int>(blocks));
  return check_launch("encode_groups_kernel");
}

}  // extern "C"
