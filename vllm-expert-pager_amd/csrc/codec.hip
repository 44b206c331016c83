// Batched GPU expansion of compressed fp8 rows (format of codec.py:1-41).
//
// One 64-lane wave decodes TWO 32-lane groups side by side (lanes 0-31 and
// 32-63). Each lane owns one chunk and keeps the last two Huffman words it
// loaded as a 64-bit funnel {hi, lo} with a bit position pos, where the
// reference's fill level is 64 - pos: the refill rule "fewer than LIMIT bits
// left" (codec.py:227-237) becomes pos > 64 - LIMIT. Refilling lanes of a
// group take consecutive words from the group's read position; the offset
// of a lane is the popcount of refilling lanes below it in its half of the
// wave ballot (mbcnt), so the word order is exactly the encoder's
// (symbol index, lane) refill order. The group's Huffman words are staged
// in LDS once (coalesced), the 512-entry LUT is split into a length table
// and a pre-shifted exponent table in LDS, and the sign/mantissa nibbles are
// read as coalesced 32-bit words, 8 values each.
#include "common.h"

namespace xp {
namespace {

constexpr int kThreads = 256;                    // 4 waves
constexpr int kGroupsPerBlock = 2 * kThreads / 64;  // 8
constexpr int kCapWords = 1536;                  // LDS staging per group (6 KiB)
constexpr int kLimit = XP_LIMIT;

struct NameDev {
  const uint8_t* stg;
  int64_t pitch;
  int64_t stg_rows;
  uint8_t* dst;
  int64_t dst_rows;
  int64_t N;
  int G;
  int blocks;  // workgroups per row for this name
};

struct DecodeArgs {
  const int64_t* todo;
  int K;
  int E;
  const int64_t* dst_row;
  const int64_t* cache_row;
  const uint8_t* lut;
  int num_names;
  NameDev names[2];
  const int64_t* skip;
  int chunk;
  int blocks_per_row;
};

// Sign + mantissa of 8 values (one nibble word) placed in their output bytes:
// byte k = (s_k & 8) << 4 | (s_k & 7). The exponent field is left zero.
__device__ __forceinline__ void nibble_template(uint32_t x, uint32_t& t_lo, uint32_t& t_hi) {
  const uint32_t ev = (x & 0x07070707u) | ((x << 4) & 0x80808080u);  // nibbles 0,2,4,6
  const uint32_t od = ((x >> 4) & 0x07070707u) | (x & 0x80808080u);  // nibbles 1,3,5,7
  t_lo = __builtin_amdgcn_perm(od, ev, 0x05010400u);
  t_hi = __builtin_amdgcn_perm(od, ev, 0x07030602u);
}

template <bool kLds>
__device__ __forceinline__ void decode_lanes(const uint32_t* __restrict__ words, int64_t nwords_limit,
                                             const uint32_t* __restrict__ nib, uint2* __restrict__ out, int msteps,
                                             bool valid, bool upper, const uint8_t* s_len, const uint8_t* s_sym) {
  uint32_t lo = 0, hi = 0;
  uint32_t pos = valid ? 64u : 0u;  // 64: nothing loaded yet, so the first step refills
  uint32_t rp = 0;                  // words of this group consumed so far (uniform per half)
  uint32_t x_next = valid ? nib[0] : 0u;
  for (int m = 0; m < msteps; ++m) {
    const uint32_t x = x_next;
    if (valid && m + 1 < msteps) x_next = nib[(m + 1) * 32];
    uint32_t o_lo, o_hi;
    nibble_template(x, o_lo, o_hi);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool refill = valid && pos > 64u - kLimit;
      const unsigned long long mask = __ballot(refill);
      const uint32_t c_lo = __popc(static_cast<uint32_t>(mask));
      const uint32_t c_hi = __popc(static_cast<uint32_t>(mask >> 32));
      if (refill) {
        const uint32_t pre = lane_prefix(mask) - (upper ? c_lo : 0u);
        uint32_t w;
        if (kLds) {
          w = words[rp + pre];
        } else {
          int64_t idx = static_cast<int64_t>(rp + pre);
          if (idx >= nwords_limit) idx = nwords_limit - 1;
          w = nwords_limit > 0 ? words[idx] : 0u;
        }
        lo = hi;
        hi = w;
        pos -= 32u;
      }
      rp += upper ? c_hi : c_lo;
      const uint64_t buf = (static_cast<uint64_t>(hi) << 32) | lo;
      const uint32_t idx = static_cast<uint32_t>(buf >> (pos & 63u)) & (XP_LUT_BYTES - 1);
      const uint32_t len = s_len[idx];
      const uint32_t sym = s_sym[idx];
      pos += valid ? len : 0u;
      if (k < 4)
        o_lo |= sym << (8 * k);
      else
        o_hi |= sym << (8 * (k - 4));
    }
    if (valid) out[m] = make_uint2(o_lo, o_hi);
  }
}

__global__ void __launch_bounds__(kThreads) decode_kernel(DecodeArgs a) {
  __shared__ uint8_t s_len[XP_LUT_BYTES];
  __shared__ uint8_t s_sym[XP_LUT_BYTES];
  __shared__ uint32_t s_words[kGroupsPerBlock][kCapWords];

  const int j = blockIdx.x / a.blocks_per_row;
  int r = blockIdx.x % a.blocks_per_row;
  const int name = r < a.names[0].blocks ? 0 : 1;
  if (name == 1) r -= a.names[0].blocks;
  const NameDev& nm = a.names[name];

  // Which expert, and whether it needs expanding (codec.py:263-277).
  const int64_t e = a.todo[j];
  bool active = e >= 0 && e < a.E;
  if (active && a.skip)
    for (int k = 0; k < a.K; ++k) active = active && a.skip[k] != e;
  if (!active || a.cache_row[e] >= 0) return;
  const int64_t drow = a.dst_row[e] > 0 ? a.dst_row[e] : 0;
  if (drow >= nm.dst_rows || j >= nm.stg_rows) return;

  const int tid = threadIdx.x;
  const uint8_t* lut = a.lut + (e * a.num_names + name) * XP_LUT_BYTES;
  for (int i = tid; i < XP_LUT_BYTES; i += kThreads) {
    const uint32_t ent = lut[i];
    s_len[i] = static_cast<uint8_t>(ent & 15u);
    s_sym[i] = static_cast<uint8_t>((ent >> 4) << 3);
  }

  const int wave = tid >> 6, lane = tid & 63;
  const bool upper = lane >= 32;
  const int li = lane & 31;
  const int gl = wave * 2 + (upper ? 1 : 0);  // group slot within the block
  const int g = r * kGroupsPerBlock + gl;
  const bool valid = g < nm.G;

  const int G = nm.G;
  const uint32_t* rec = reinterpret_cast<const uint32_t*>(nm.stg + int64_t(j) * nm.pitch);
  const int64_t nib_words = nm.N / 8;
  const int64_t huff_off = (G + 1) + nib_words;                 // in words
  const int64_t maxw = nm.pitch / 4 - huff_off;                 // Huffman words that fit in the record
  int64_t gs = 0, ge = 0;
  if (valid && maxw > 0) {
    gs = rec[g];
    ge = rec[g + 1];
    gs = gs < 0 ? 0 : (gs > maxw ? maxw : gs);
    ge = ge < gs ? gs : (ge > maxw ? maxw : ge);
  }
  const int64_t count = ge - gs;
  const uint32_t* huff = rec + huff_off + gs;

  // Stage the group's words in LDS when both groups of the wave fit.
  const bool fits = !valid || count <= kCapWords;
  const bool lds_mode = __ballot(!fits) == 0;
  if (lds_mode && valid)
    for (int64_t i = li; i < count; i += 32) s_words[gl][i] = huff[i];
  __syncthreads();

  const uint32_t* nib = rec + (G + 1) + (int64_t(g) * (a.chunk / 8)) * 32 + li;
  uint2* out = reinterpret_cast<uint2*>(nm.dst + drow * nm.N + (int64_t(g) * 32 + li) * a.chunk);
  const int msteps = a.chunk / 8;
  if (lds_mode)
    decode_lanes<true>(s_words[gl], count, nib, out, msteps, valid, upper, s_len, s_sym);
  else
    decode_lanes<false>(huff, count, nib, out, msteps, valid, upper, s_len, s_sym);
}

}  // namespace
}  // namespace xp

using namespace xp;

extern "C" {

int xp_decode_rows(const int64_t* todo, int64_t K, int64_t num_experts, const int64_t* dst_row,
                   const int64_t* cache_row, const uint8_t* lut, const xp_decode_name* names, int num_names,
                   const int64_t* skip, int64_t chunk, void* stream) {
  XP_REQUIRE(K >= 0 && K <= (1 << 20), "xp_decode_rows: K=%lld", (long long)K);
  XP_REQUIRE(num_names >= 1 && num_names <= 2 && names, "xp_decode_rows: %d names (1 or 2)", num_names);
  XP_REQUIRE(chunk >= 8 && chunk % 8 == 0 && chunk <= 4096, "xp_decode_rows: chunk=%lld (multiple of 8)",
             (long long)chunk);
  XP_REQUIRE(num_experts >= 1, "xp_decode_rows: num_experts=%lld", (long long)num_experts);
  if (K == 0) return XP_OK;
  XP_REQUIRE(todo && dst_row && cache_row && lut, "xp_decode_rows: null index tensor");
  DecodeArgs a{};
  a.todo = todo;
  a.K = static_cast<int>(K);
  a.E = static_cast<int>(num_experts);
  a.dst_row = dst_row;
  a.cache_row = cache_row;
  a.lut = lut;
  a.num_names = num_names;
  a.skip = skip;
  a.chunk = static_cast<int>(chunk);
  int per_row = 0;
  for (int n = 0; n < num_names; ++n) {
    const xp_decode_name& s = names[n];
    const int64_t group = chunk * XP_LANES;
    XP_REQUIRE(s.row_bytes > 0 && s.row_bytes % group == 0,
               "xp_decode_rows: name %d row of %lld values is not a multiple of %lld", n, (long long)s.row_bytes,
               (long long)group);
    const int64_t G = s.row_bytes / group;
    XP_REQUIRE(s.pitch % 4 == 0 && s.pitch >= 4 * (G + 1) + s.row_bytes / 2,
               "xp_decode_rows: name %d pitch %lld cannot hold the record header", n, (long long)s.pitch);
    XP_REQUIRE(s.stg && s.dst, "xp_decode_rows: name %d has a null buffer", n);
    XP_REQUIRE(aligned16(s.stg) && aligned16(s.dst), "xp_decode_rows: name %d buffers must be 16-byte aligned", n);
    a.names[n] = NameDev{static_cast<const uint8_t*>(s.stg),
                         s.pitch,
                         s.stg_rows,
                         static_cast<uint8_t*>(s.dst),
                         s.dst_rows,
                         s.row_bytes,
                         static_cast<int>(G),
                         static_cast<int>((G + kGroupsPerBlock - 1) / kGroupsPerBlock)};
    per_row += a.names[n].blocks;
  }
  if (num_names == 1) a.names[1] = a.names[0];
  a.blocks_per_row = per_row;
  const int64_t grid = K * per_row;
  XP_REQUIRE(grid <= (int64_t(1) << 31) - 1, "xp_decode_rows: grid too large");
  hipLaunchKernelGGL(decode_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, as_stream(stream), a);
  return check_launch("decode_kernel");
}

}  // extern "C"
