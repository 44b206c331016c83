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

// Huffman lengths of 16 weighted symbols (ties broken by node id).
__host__ __device__ inline void huffman_lengths(const double* counts, int32_t* lengths) {
  double c[kSyms];
  int id[kSyms];
  uint32_t members[kSyms];  // bit s set: symbol s is under the node
  int n = kSyms;
  for (int i = 0; i < kSyms; ++i) {
    c[i] = counts[i];
    id[i] = i;
    members[i] = 1u << i;
    lengths[i] = 0;
  }
  int next_id = kSyms;
  while (n > 1) {
    double pc[2];
    uint32_t pm[2];
    for (int t = 0; t < 2; ++t) {
      int best = 0;
      for (int i = 1; i < n; ++i)
        if (c[i] < c[best] || (c[i] == c[best] && id[i] < id[best])) best = i;
      pc[t] = c[best];
      pm[t] = members[best];
      --n;  // the last node moves into the picked one's place
      c[best] = c[n];
      id[best] = id[n];
      members[best] = members[n];
    }
    const uint32_t m = pm[0] | pm[1];
    for (int s = 0; s < kSyms; ++s)
      if (m & (1u << s)) ++lengths[s];
    c[n] = pc[0] + pc[1];
    id[n] = next_id++;
    members[n] = m;
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

// Canonical codes in (length, symbol) order, bit-reversed.
__host__ __device__ inline void canonical_codes(const int32_t* lengths, int32_t* codes) {
  int order[kSyms];
  for (int i = 0; i < kSyms; ++i) order[i] = i;
  for (int i = 1; i < kSyms; ++i)  // insertion sort by (length, symbol)
    for (int k = i; k > 0 && (lengths[order[k]] < lengths[order[k - 1]] ||
                              (lengths[order[k]] == lengths[order[k - 1]] && order[k] < order[k - 1]));
         --k) {
      const int t = order[k];
      order[k] = order[k - 1];
      order[k - 1] = t;
    }
  uint32_t canon[kSyms] = {0};
  uint32_t code = 0;
  for (int i = 0; i < kSyms; ++i) {
    const int s = order[i];
    if (i) code = (code + 1) << (lengths[s] - lengths[order[i - 1]]);
    canon[s] = code;
  }
  for (int s = 0; s < kSyms; ++s) {
    uint32_t rev = 0;
    for (int b = 0; b < lengths[s]; ++b)
      if (canon[s] & (1u << b)) rev |= 1u << (lengths[s] - 1 - b);
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
