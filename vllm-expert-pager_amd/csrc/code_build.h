// Code construction of the fp8 exponent Huffman row format, shared by the
// host encoder (codec_host.cpp) and the GPU encoder (encode.hip).
//
// The code is fixed by the format (codec.py:61-114):
//   - length-limited Huffman lengths: merge the two lightest (count, id)
//     nodes, new ids from 16 up; if a length exceeds LIMIT, raise every count
//     to sum / 2^(LIMIT - k) and retry (codec.py:61-87);
//   - canonical codes in (length, symbol) order, stored bit-reversed (the
//     stream is read least significant bit first), and a 512-entry LUT of
//     (symbol << 4) | length (codec.py:90-114).
// Counts are doubles and every step is plain IEEE arithmetic, so host and
// device give the same lengths.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/xp.h"

namespace xp {
namespace code {

constexpr int kSyms = 16;

// Huffman lengths of 16 weighted symbols (ties broken by node id). Every
// array is indexed by loop constants only (selects instead of dynamic
// indexing), so on the GPU it stays in registers rather than scratch memory.
__host__ __device__ inline void huffman_lengths(const double* counts, int32_t* lengths) {
  double c[kSyms];
  int id[kSyms];
  uint32_t members[kSyms];  // bit s set: symbol s is under the node
#pragma unroll
  for (int i = 0; i < kSyms; ++i) {
    c[i] = counts[i];
    id[i] = i;
    members[i] = 1u << i;
    lengths[i] = 0;
  }
  int n = kSyms, next_id = kSyms;
  for (int step = 0; step < kSyms - 1; ++step) {  // 16 nodes merge into one
    double pc[2];
    uint32_t pm[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      // The lightest of the n live nodes, the lower id on a tie.
      int best = 0, bid = id[0];
      double bc = c[0];
      uint32_t bm = members[0];
#pragma unroll
      for (int i = 1; i < kSyms; ++i) {
        const bool take = i < n && (c[i] < bc || (c[i] == bc && id[i] < bid));
        best = take ? i : best;
        bc = take ? c[i] : bc;
        bid = take ? id[i] : bid;
        bm = take ? members[i] : bm;
      }
      pc[t] = bc;
      pm[t] = bm;
      --n;  // the last node moves into the picked one's place
      double lc = 0.0;
      int lid = 0;
      uint32_t lm = 0;
#pragma unroll
      for (int i = 0; i < kSyms; ++i)
        if (i == n) {
          lc = c[i];
          lid = id[i];
          lm = members[i];
        }
#pragma unroll
      for (int i = 0; i < kSyms; ++i)
        if (i == best) {
          c[i] = lc;
          id[i] = lid;
          members[i] = lm;
        }
    }
    const uint32_t m = pm[0] | pm[1];
#pragma unroll
    for (int s = 0; s < kSyms; ++s) lengths[s] += static_cast<int32_t>((m >> s) & 1u);
#pragma unroll
    for (int i = 0; i < kSyms; ++i)
      if (i == n) {
        c[i] = pc[0] + pc[1];
        id[i] = next_id;
        members[i] = m;
      }
    ++next_id;
    ++n;
  }
}

// Lengths of the row's code from its exponent histogram, at most LIMIT.
__host__ __device__ inline void code_lengths(const int64_t* hist, int32_t* lengths) {
  double counts[kSyms];
  for (int i = 0; i < kSyms; ++i) counts[i] = static_cast<double>(hist[i] > 1 ? hist[i] : 1);
  for (int k = 0;; ++k) {
    if (k > 0) {
      // k never passes LIMIT: at k = LIMIT every count is the sum, and 16
      // equal counts give length 4.
      double sum = 0.0;
      for (int i = 0; i < kSyms; ++i) sum += counts[i];
      const double floor_c = sum / static_cast<double>(1 << (XP_LIMIT - k));
      for (int i = 0; i < kSyms; ++i) counts[i] = counts[i] > floor_c ? counts[i] : floor_c;
    }
    huffman_lengths(counts, lengths);
    int mx = 0;
    for (int i = 0; i < kSyms; ++i) mx = lengths[i] > mx ? lengths[i] : mx;
    if (mx <= XP_LIMIT) return;
  }
}

// Canonical codes in (length, symbol) order, bit-reversed: the first code
// of length L is (first code of L - 1 + count of length L - 1) << 1, and
// symbols of one length take consecutive codes in symbol order. Loop
// constants index every array (see huffman_lengths).
__host__ __device__ inline void canonical_codes(const int32_t* lengths, int32_t* codes) {
  uint32_t first[XP_LIMIT + 1];
  uint32_t code = 0, prev = 0;
#pragma unroll
  for (int L = 1; L <= XP_LIMIT; ++L) {
    code = (code + prev) << 1;
    first[L] = code;
    prev = 0;
#pragma unroll
    for (int s = 0; s < kSyms; ++s) prev += lengths[s] == L ? 1u : 0u;
  }
  first[0] = 0;
#pragma unroll
  for (int s = 0; s < kSyms; ++s) {
    const int L = lengths[s];
    uint32_t canon = 0;
#pragma unroll
    for (int k = 1; k <= XP_LIMIT; ++k) canon = k == L ? first[k] : canon;
#pragma unroll
    for (int t = 0; t < s; ++t) canon += lengths[t] == L ? 1u : 0u;
    uint32_t rev = 0;
#pragma unroll
    for (int b = 0; b < XP_LIMIT; ++b)
      if (b < L && (canon & (1u << b))) rev |= 1u << (L - 1 - b);
    codes[s] = static_cast<int32_t>(rev);
  }
}

// LUT entry of the 9-bit window x: the symbol whose code is x's low bits,
// (symbol << 4) | length; -1 if none (a code set with Kraft sum < 1).
__host__ __device__ inline int lut_entry(const int32_t* lengths, const int32_t* codes, int x) {
  for (int s = 0; s < kSyms; ++s) {
    const int n = lengths[s];
    if ((x & ((1 << n) - 1)) == codes[s]) return (s << 4) | n;
  }
  return -1;
}

}  // namespace code
}  // namespace xp
