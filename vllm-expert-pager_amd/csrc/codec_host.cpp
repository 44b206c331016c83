// Host encoder of the fp8 exponent Huffman row format (codec.py:1-41, 61-198).
//
// The record layout, the code construction and the Huffman word order are
// fixed by the format, so this follows the reference's rules step for step:
//   - the code (lengths, canonical bit-reversed codes, LUT) as in
//     code_build.h (codec.py:61-114);
//   - record = int32 gstart[G+1] | sign/mantissa nibble words in
//     (group, word, lane) order | Huffman words per group in refill order
//     (codec.py:125-193).
// The refill order is produced by running the decoder's refill rule (a word
// whenever fewer than LIMIT bits are buffered) over each chunk's code
// lengths, which yields the same (symbol index, lane) order as the
// reference's searchsorted formulation.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "code_build.h"

namespace xp {
int fail(int code, const char* fmt, ...);
}

namespace {

constexpr int kSyms = xp::code::kSyms;

int build_code(const int64_t* hist, int32_t* lengths, int32_t* codes, uint8_t* lut) {
  xp::code::code_lengths(hist, lengths);
  xp::code::canonical_codes(lengths, codes);
  int16_t table[XP_LUT_BYTES];
  for (int i = 0; i < XP_LUT_BYTES; ++i) table[i] = -1;
  for (int s = 0; s < kSyms; ++s) {
    const int n = lengths[s];
    for (int h = 0; h < (1 << (XP_LIMIT - n)); ++h) {
      const int x = codes[s] | (h << n);
      if (table[x] >= 0) return xp::fail(XP_E_ARG, "codes are not prefix-free");
      table[x] = static_cast<int16_t>((s << 4) | n);
    }
  }
  for (int i = 0; i < XP_LUT_BYTES; ++i) {
    if (table[i] < 0) return xp::fail(XP_E_ARG, "codes do not fill the LUT (Kraft sum < 1)");
    lut[i] = static_cast<uint8_t>(table[i]);
  }
  return XP_OK;
}

}  // namespace

extern "C" {

int xp_code_build(const int64_t* hist, int32_t* lengths, int32_t* codes, uint8_t* lut) {
  if (!hist || !lengths || !codes || !lut) return xp::fail(XP_E_ARG, "xp_code_build: null argument");
  return build_code(hist, lengths, codes, lut);
}

int xp_encode_row(const uint8_t* raw, int64_t n, int64_t chunk, uint8_t* record, int64_t pitch, uint8_t* lut,
                  int64_t* needed) {
  if (!raw || !record || !lut || n <= 0 || pitch <= 0 || chunk < 8 || chunk % 8)
    return xp::fail(XP_E_ARG, "xp_encode_row: bad arguments");
  const int64_t group = chunk * XP_LANES;
  if (n % group) return xp::fail(XP_E_SHAPE, "row of %lld values is not a multiple of %lld", (long long)n, (long long)group);
  const int64_t C = n / chunk, G = n / group;

  int64_t hist[kSyms] = {0};
  for (int64_t i = 0; i < n; ++i) ++hist[(raw[i] >> 3) & 15];
  int32_t lengths[kSyms], codes[kSyms];
  int rc = build_code(hist, lengths, codes, lut);
  if (rc) return rc;

  // Per chunk: the bit stream of its codes as 32-bit words, and the symbol
  // index at which the decoder loads each word.
  std::vector<std::vector<uint32_t>> words(static_cast<size_t>(C));
  std::vector<std::vector<int32_t>> at(static_cast<size_t>(C));
  int64_t total_words = 0;
  for (int64_t c = 0; c < C; ++c) {
    const uint8_t* v = raw + c * chunk;
    std::vector<uint32_t>& w = words[static_cast<size_t>(c)];
    std::vector<int32_t>& a = at[static_cast<size_t>(c)];
    uint64_t bit = 0;
    int64_t level = 0;
    for (int64_t i = 0; i < chunk; ++i) {
      if (level < XP_LIMIT) {  // the decoder refills before symbol i
        a.push_back(static_cast<int32_t>(i));
        level += 32;
      }
      const int s = (v[i] >> 3) & 15;
      const int len = lengths[s];
      const uint64_t code = static_cast<uint64_t>(codes[s]);
      const size_t wi = static_cast<size_t>(bit >> 5);
      const unsigned sh = static_cast<unsigned>(bit & 31);
      if (w.size() < wi + 2) w.resize(wi + 2, 0u);
      w[wi] |= static_cast<uint32_t>(code << sh);
      if (sh + len > 32) w[wi + 1] |= static_cast<uint32_t>(code >> (32 - sh));
      bit += static_cast<uint64_t>(len);
      level -= len;
    }
    w.resize(a.size());  // one word per refill
    total_words += static_cast<int64_t>(a.size());
  }

  const int64_t head = 4 * (G + 1) + n / 2;
  const int64_t nbytes = head + 4 * total_words;
  if (needed) *needed = nbytes;
  if (nbytes > pitch)
    return xp::fail(XP_E_PITCH, "compressed row is %lld B, pitch is %lld B; VLLM_EXPERT_PAGER_PITCH must be at least %.4f",
                    (long long)nbytes, (long long)pitch, static_cast<double>(nbytes) / static_cast<double>(n));

  std::memset(record, 0, static_cast<size_t>(pitch));
  int32_t* gstart = reinterpret_cast<int32_t*>(record);
  uint32_t* fixed = reinterpret_cast<uint32_t*>(record + 4 * (G + 1));
  uint32_t* huff = reinterpret_cast<uint32_t*>(record + head);
  const int64_t mwords = chunk / 8;
  // Sign + mantissa nibbles: word (g, m, lane) holds values 8m..8m+7 of chunk
  // g*LANES + lane, value k in bits 4k..4k+3.
  for (int64_t g = 0; g < G; ++g)
    for (int64_t m = 0; m < mwords; ++m)
      for (int l = 0; l < XP_LANES; ++l) {
        const uint8_t* v = raw + ((g * XP_LANES + l) * chunk) + 8 * m;
        uint32_t word = 0;
        for (int k = 0; k < 8; ++k) {
          const uint32_t sm = (static_cast<uint32_t>(v[k] >> 7) << 3) | (v[k] & 7u);
          word |= sm << (4 * k);
        }
        fixed[(g * mwords + m) * XP_LANES + l] = word;
      }
  // Huffman words of each group in (symbol index, lane) order.
  int64_t pos = 0;
  for (int64_t g = 0; g < G; ++g) {
    gstart[g] = static_cast<int32_t>(pos);
    size_t next[XP_LANES] = {0};
    for (int64_t i = 0; i < chunk; ++i)
      for (int l = 0; l < XP_LANES; ++l) {
        const size_t c = static_cast<size_t>(g * XP_LANES + l);
        if (next[l] < at[c].size() && at[c][next[l]] == i) huff[pos++] = words[c][next[l]++];
      }
  }
  gstart[G] = static_cast<int32_t>(pos);
  return XP_OK;
}

}  // extern "C"
