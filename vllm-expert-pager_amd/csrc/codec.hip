// Batched GPU expansion of compressed fp8 rows (format of codec.py:1-41).
//
// One 64-lane wave decodes TWO 32-lane groups side by side (lanes 0-31 and
// 32-63). Each lane owns one chunk and keeps the last two Huffman words it
// loaded as a 64-bit funnel {hi, lo} with a bit position p (kept as p - 1);
// the reference's fill level is 64 - p, so its refill rule "fewer than LIMIT
// bits left" (codec.py:227-237) becomes p > 64 - LIMIT. At each symbol the
// refilling lanes of a group take consecutive words from the group's read
// position, a lane's offset being the number of refilling lanes below it in
// its half of the wave ballot (mbcnt) -- exactly the encoder's
// (symbol index, lane) word order.
//
// Memory: the group's Huffman words stream through a 256-word ring in LDS
// (plus a 224-word mirror of its head, so a step's reads never wrap), kept
// at least 192 words ahead of the reads: each 16-symbol step issues a
// coalesced 64-word load at its start and lands it at its end. The
// 512-entry LUT is a 16-bit table in LDS (length, pre-shifted exponent); the
// sign/mantissa nibbles arrive as coalesced 32-bit words (8 values each),
// prefetched a step ahead. Output bytes are gathered per lane and stored
// through a lane transpose in runs of 128 bytes (flush16). The kernel is held
// to 64 VGPRs, so that 8 waves share each SIMD.
#include "common.h"

#include <type_traits>

namespace xp {
namespace {

constexpr int kThreads = 256;                  // 4 waves
constexpr int kGroupsPerBlock = 2 * kThreads / 64;  // 8: lanes 0-31 and 32-63 of each wave
constexpr uint32_t kRing = 256;                // ring words per group
constexpr uint32_t kHalf = 16;                 // symbols between ring maintenance (two nibble words)
// Words a group may consume in kHalf symbols. A lane refills only when fewer
// than LIMIT bits are left and then holds at least 32; a symbol takes at most
// LIMIT bits, so its next refill is at least ceil((32 - LIMIT + 1) / LIMIT) = 3
// symbols later: at most ceil(kHalf / 3) refills per lane in a half.
constexpr uint32_t kAhead = 32 * ((kHalf + 2) / 3);
constexpr uint32_t kMirror = kAhead + 32;      // reads of a half never wrap
constexpr uint32_t kRingPad = kRing + kMirror;
constexpr uint32_t kFetch = 64;                // words requested per half-iteration (two per lane)
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
  const uint32_t* scale;  // reading the RAM tier: scale rows by expert, copied to
  uint32_t* scale_dst;    // scale_dst[dst_row] (scale_words 4-byte words each)
  int scale_words;
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
  const int64_t* src_row;  // non-null: expert e's record is stg row src_row[e] + base, else row j
  int64_t base;
};

// Sign + mantissa of 8 values (one nibble word) in their output bytes:
// byte k = (s_k & 8) << 4 | (s_k & 7); the exponent field is left zero.
__device__ __forceinline__ uint2 nibble_template(uint32_t x) {
  const uint32_t ev = (x & 0x07070707u) | ((x << 4) & 0x80808080u);  // nibbles 0,2,4,6
  const uint32_t od = ((x >> 4) & 0x07070707u) | (x & 0x80808080u);  // nibbles 1,3,5,7
  return make_uint2(__builtin_amdgcn_perm(od, ev, 0x05010400u), __builtin_amdgcn_perm(od, ev, 0x07030602u));
}

// Ring of one group: word w of the group's stream sits in slot w % kRing,
// and also in slot w % kRing + kRing when that slot is below kMirror.
__device__ __forceinline__ void ring_put(uint32_t* ring, uint32_t w_index, uint32_t value) {
  const uint32_t s = w_index & (kRing - 1);
  ring[s] = value;
  if (s < kMirror) ring[s + kRing] = value;
}

// One lane's stream: a chunk of the group of this lane's half.
struct Chain {
  uint64_t buf;      // {hi, lo}: the last two words loaded
  uint32_t pos;      // next bit in buf minus one (the window shift then scales the LUT
                     // index to a byte offset); the fill level is 63 - pos. At least 1
                     // bit is always consumed before a window is read, so it never wraps.
  uint32_t b_val0, b_val1;  // this lane's words of the request in flight
  uint32_t x_next;   // nibble word of the next iteration
  uint32_t x_next1;  // and the one after it, when both are fetched an iteration ahead
  uint32_t wsrc;     // byte offset in the record of the group's word li (this lane's column)
  uint32_t nib;      // byte offset in the record of this lane's first nibble word
  uint32_t* ring;
};

// The ring state of the wave's two groups (index h: lanes 32h .. 32h + 31).
// Every field is the same in all lanes, so it lives in scalar registers and
// its upkeep is scalar work; a lane takes its half's value, with one
// bit-field extract from a pair packed in 16-bit halves, only where an
// address needs it. Word indices stay below 2^16: a group's word count is
// clamped to 65535, above the words any group can consume (chunk <= 4096
// symbols per lane of at most LIMIT bits: 32 * 4096 * 9 / 32 words, plus
// one refill per lane).
struct Rings {
  uint32_t rp[2];     // words of the group consumed
  uint32_t fe[2];     // the ring holds words [rp, fe)
  uint32_t q[2];      // words requested so far (landed or in flight)
  uint32_t count[2];  // Huffman words of the group
  uint32_t base[2];   // LDS word address (byte address / 4) of the group's ring
  uint32_t bb[2];     // first word of the request in flight
  uint32_t bn[2];     // and its word count
  uint32_t ab0[2];    // LDS word address of word rp at the half's start
};

// Minimum of two wave-uniform values on the scalar unit. Written as an
// instruction because the compiler otherwise fuses two minimums into a
// vector min3 and reads the result back into a scalar register.
__device__ __forceinline__ uint32_t smin(uint32_t a, uint32_t b) {
  uint32_t r;
  asm("s_min_u32 %0, %1, %2" : "=s"(r) : "s"(a), "s"(b));
  return r;
}

// lo | hi << 16 for wave-uniform values below 2^16, as one scalar pack.
__device__ __forceinline__ uint32_t spack(uint32_t lo, uint32_t hi) {
  uint32_t r;
  asm("s_pack_ll_b32_b16 %0, %1, %2" : "=s"(r) : "s"(lo), "s"(hi));
  return r;
}

// This lane's value of a per-group pair (both below 2^16).
__device__ __forceinline__ uint32_t lane_half(const uint32_t (&v)[2], uint32_t half_shift) {
  return __builtin_amdgcn_ubfe(spack(v[0], v[1]), half_shift, 16u);
}

// Start of a half-iteration: make sure each ring holds the next kAhead words,
// then request up to kFetch more (landed at the end of this half).
__device__ __forceinline__ void half_begin(Rings& r, Chain& c, uint32_t li, bool upper, uint32_t half_shift,
                                           __amdgpu_buffer_rsrc_t rec) {
  bool slow = false;
#pragma unroll
  for (int h = 0; h < 2; ++h) slow = slow || (r.fe[h] < r.count[h] && r.fe[h] < r.rp[h] + kAhead);
  if (slow) {  // the stream outran the requests: this lane's group, 32 words at a time
    uint32_t fe = upper ? r.fe[1] : r.fe[0];
    const uint32_t count = upper ? r.count[1] : r.count[0];
    const uint32_t lim = (upper ? r.rp[1] : r.rp[0]) + kAhead;
    while (fe < count && fe < lim) {
      const uint32_t w = fe + li;
      const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(rec, c.wsrc + 4u * fe, 0, 0);
      if (w < count) ring_put(c.ring, w, v);
      fe = fe + 32 < count ? fe + 32 : count;
    }
    r.fe[0] = __builtin_amdgcn_readlane(fe, 0);
    r.fe[1] = __builtin_amdgcn_readlane(fe, 32);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    r.q[h] = r.q[h] > r.fe[h] ? r.q[h] : r.fe[h];
    const uint32_t room = r.rp[h] + kRing - r.q[h];
    const uint32_t want = r.count[h] - r.q[h];
    const uint32_t n = smin(smin(want, room), kFetch);
    r.bb[h] = r.q[h];
    r.bn[h] = n;
    r.q[h] += n;
    r.ab0[h] = r.base[h] + (r.rp[h] & (kRing - 1));
  }
  // Reads past the group's words return other bytes of the record (never
  // used), past the record zeros: the buffer's range check bounds them.
  const uint32_t a = c.wsrc + 4u * lane_half(r.bb, half_shift);
  c.b_val0 = __builtin_amdgcn_raw_buffer_load_b32(rec, a, 0, 0);
  c.b_val1 = __builtin_amdgcn_raw_buffer_load_b32(rec, a + 128u, 0, 0);
}

// End of a half-iteration: offs holds each group's next unread ring word
// address (low | high << 16); land the request in the ring (its slots hold
// words already consumed).
__device__ __forceinline__ void half_end(Rings& r, Chain& c, uint32_t li, uint32_t half_shift, uint32_t offs) {
#pragma unroll
  for (int h = 0; h < 2; ++h) r.rp[h] += ((offs >> (16 * h)) & 0xFFFFu) - r.ab0[h];
  const uint32_t bb = lane_half(r.bb, half_shift), bn = lane_half(r.bn, half_shift);
  if (li < bn) ring_put(c.ring, bb + li, c.b_val0);
  if (li + 32 < bn) ring_put(c.ring, bb + 32 + li, c.b_val1);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t landed = r.bb[h] + r.bn[h];
    r.fe[h] = r.fe[h] > landed ? r.fe[h] : landed;
  }
}

// mask[lane] ? if1 : if0, as one v_cndmask. Written as an instruction so
// that the compiler keeps the step branch-free instead of turning the
// select back into a branch around the ring read.
__device__ __forceinline__ uint32_t lane_select(unsigned long long mask, uint32_t if0, uint32_t if1) {
  uint32_t r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(if0), "v"(if1), "s"(mask));
  return r;
}

// pos + (byte 0 of e) as one byte-select add. Volatile, like the byte
// selects of quad(), so that the compiler keeps those where they are written.
__device__ __forceinline__ uint32_t add_byte0(uint32_t pos, uint32_t e) {
  uint32_t r;
  asm volatile("v_add_u32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0 src1_sel:DWORD"
      : "=v"(r) : "v"(e), "v"(pos));
  return r;
}

// One symbol of one stream, without branches: every lane reads a ring word
// at its refill address and keeps it only if it refills. s_lut holds
// len | (symbol << 3) << 8 per 9-bit code, followed by the 64-byte position
// table: entry p is p - 32 for a position that refills (p > 63 - LIMIT),
// else p. Reading it replaces a select and an add per symbol by one LDS
// read issued beside the ring read. offs packs the LDS word
// addresses (byte address / 4) of the next unread ring word of the groups of
// the lower and upper half-wave (low | high << 16; both below 2^16):
// wave-uniform, so it advances in a scalar register, by one 16-bit pack and
// one add.
// A lane's refill word is (refilling lanes below it in its half) words on;
// mbcnt over the whole ballot also counts, for an upper-half lane, every
// refilling lane of the lower half, so that half's base is lowered by as
// many words and one bit-field extract picks each lane's base.
__device__ __forceinline__ uint32_t decode_symbol(uint64_t& buf, uint32_t& pos, uint32_t& offs, uint32_t half_shift,
                                                  const uint16_t* s_lut) {
  // pos is the next bit's index minus one (see Chain::pos); pr is the
  // position after this symbol's refill (pos - 32 in refilling lanes).
  const uint32_t pr = reinterpret_cast<const uint8_t*>(s_lut)[2 * XP_LUT_BYTES + pos];
  const unsigned long long mask = __builtin_amdgcn_ballot_w64(pos > 63u - kLimit);
  const uint32_t m_lo = static_cast<uint32_t>(mask), m_hi = static_cast<uint32_t>(mask >> 32);
  const uint32_t n_lo = static_cast<uint32_t>(__popc(m_lo)), n_hi = static_cast<uint32_t>(__popc(m_hi));
  const uint32_t bases = offs - (n_lo << 16);  // the upper half's base lowered by n_lo words
  const uint32_t below = __builtin_amdgcn_mbcnt_hi(m_hi, __builtin_amdgcn_mbcnt_lo(m_lo, 0u));
  const uint32_t addr = (__builtin_amdgcn_ubfe(bases, half_shift, 16u) + below) << 2;
  const uint32_t w = *reinterpret_cast<const __attribute__((address_space(3))) uint32_t*>(addr);
  offs += spack(n_lo, n_hi);
  const uint32_t lo = static_cast<uint32_t>(buf), hi = static_cast<uint32_t>(buf >> 32);
  const uint32_t nlo = lane_select(mask, lo, hi), nhi = lane_select(mask, hi, w);
  buf = (static_cast<uint64_t>(nhi) << 32) | nlo;
  // The window's 9 bits shifted up by one: the byte offset of its 16-bit entry.
  const uint32_t e = *reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(s_lut) +
                                                          (static_cast<uint32_t>(buf >> (pr & 63u)) & (2u * XP_LUT_BYTES - 2)));
  pos = add_byte0(pr, e);
  return e;
}

// Byte select (v_perm) kept in program order with the symbol steps (all
// volatile), so that the entries it reads are dead right after it instead
// of being held for a select the compiler would defer.
__device__ __forceinline__ uint32_t sel_bytes(uint32_t hi, uint32_t lo, uint32_t sel) {
  uint32_t r;
  asm volatile("v_perm_b32 %0, %1, %2, %3" : "=v"(r) : "v"(hi), "v"(lo), "s"(sel));
  return r;
}

// Four symbols of one stream into one output word: the exponent field
// (byte 1 of each entry) of symbol k goes to byte k, joined to the sign and
// mantissa bits in tmpl. Two byte selects and a three-way OR per four
// symbols.
__device__ __forceinline__ uint32_t quad(Chain& ch, uint32_t& offs, uint32_t half_shift, const uint16_t* s_lut,
                                         uint32_t tmpl) {
  const uint32_t e0 = decode_symbol(ch.buf, ch.pos, offs, half_shift, s_lut);
  const uint32_t e1 = decode_symbol(ch.buf, ch.pos, offs, half_shift, s_lut);
  const uint32_t p01 = sel_bytes(e1, e0, 0x0c0c0501u);  // selector 0x0c gives a zero byte
  const uint32_t e2 = decode_symbol(ch.buf, ch.pos, offs, half_shift, s_lut);
  const uint32_t e3 = decode_symbol(ch.buf, ch.pos, offs, half_shift, s_lut);
  const uint32_t p23 = sel_bytes(e3, e2, 0x05010c0cu);
  uint32_t r;
  asm volatile("v_or3_b32 %0, %1, %2, %3" : "=v"(r) : "v"(p01), "v"(p23), "v"(tmpl));
  return r;
}

// One stage of the transpose of 16-byte pieces w[4j..4j+3] (j < NP) over
// sets of lanes four apart: the lanes whose bit T (2 or 3) is clear swap
// their pieces j | D with pieces j of the partner lane (this lane + 2^T),
// D = 2^(T-2). The exchange is a pair of row shifts whose bank masks write
// only the receiving lanes (a bank is lanes with equal bits 3:2).
template <int T, int NP>
__device__ __forceinline__ void butterfly(uint32_t (&w)[4 * NP]) {
  constexpr int D = 1 << (T - 2);
#pragma unroll
  for (int i = 0; i < 2 * NP; ++i) {
    const int jj = i >> 2, k = i & 3;
    const int j = ((jj & ~(D - 1)) << 1) | (jj & (D - 1));  // the pieces whose bit D is clear
    const int ia = 4 * j + k, ib = 4 * (j | D) + k;
    constexpr int kShl = 0x100 | (1 << T), kShr = 0x110 | (1 << T);  // lane i <- i + 2^T, i - 2^T
    constexpr int kClear = T == 2 ? 0x5 : 0x3, kSet = T == 2 ? 0xA : 0xC;
    const uint32_t nb = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(w[ib]), static_cast<int>(w[ia]), kShl, 0xF, kClear, false));
    const uint32_t na = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(static_cast<int>(w[ia]), static_cast<int>(w[ib]), kShr, 0xF, kSet, false));
    w[ia] = na;
    w[ib] = nb;
  }
}

// Store of a lane's last F iterations (8F bytes at byte `off` of its
// chunk, NP = F/2 pieces of 16 bytes), for F of 4 or 8 (16: flush16). For
// F = 8 the lanes of a half-wave form sets of 4 lanes four apart (lane bits
// 2 and 3); the transpose leaves set member q with piece q of each member's
// chunk, so store j of the set writes 64 contiguous bytes of member j's
// chunk: one store instruction covers 16 runs rather than 64 separate
// 16-byte pieces. Every lane takes part in the exchange; only valid streams
// store.
template <int F>
__device__ __forceinline__ void flush(uint4 (&ob)[F / 2], uint8_t* chunk0, int64_t chunk, uint32_t li, int64_t off,
                                      bool valid) {
  constexpr int NP = F / 2;
  static_assert(NP == 2 || NP == 4, "flush16 stores 16 iterations");
  if constexpr (NP == 4) {
    const uint32_t q = (li >> 2) & (NP - 1);
    uint32_t w[4 * NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      w[4 * j] = ob[j].x;
      w[4 * j + 1] = ob[j].y;
      w[4 * j + 2] = ob[j].z;
      w[4 * j + 3] = ob[j].w;
    }
    butterfly<2, NP>(w);
    butterfly<3, NP>(w);
    if (valid) {
      uint8_t* base = chunk0 + static_cast<int64_t>(li & ~(4u * NP - 4u)) * chunk + off + 16 * q;
#pragma unroll
      for (int j = 0; j < NP; ++j)
        *reinterpret_cast<uint4*>(base + 4 * j * chunk) = make_uint4(w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]);
    }
  } else {
    if (valid) {
      uint4* dst = reinterpret_cast<uint4*>(chunk0 + static_cast<int64_t>(li) * chunk + off);
#pragma unroll
      for (int i = 0; i < NP; ++i) dst[i] = ob[i];
    }
  }
}

// Store of a lane's last 16 iterations (128 bytes at byte `off` of its
// chunk, 8 pieces of 16 bytes) for the whole wave at once. The wave's 64
// lanes hold 64 consecutive chunks (the upper half's group follows the
// lower half's), starting at chunk0. Sets of eight lanes 8 apart (lane bits
// 3, 4 and 5) trade pieces in three stages: a pair of row shifts over 8
// lanes, a swap over 16 lanes and a swap over the wave's halves. Afterwards
// set member q holds piece q of each member m's run in slot m, so store m
// writes member m's whole 128-byte line per set. A half whose group is a
// spare stores nothing.
__device__ __forceinline__ void flush16(uint4 (&ob)[8], uint8_t* chunk0, int64_t chunk, uint32_t lane, int64_t off,
                                        bool valid_lo, bool valid_hi) {
  uint32_t w[32];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    w[4 * j] = ob[j].x;
    w[4 * j + 1] = ob[j].y;
    w[4 * j + 2] = ob[j].z;
    w[4 * j + 3] = ob[j].w;
  }
  // Lanes with bit 3 set trade their piece j for piece j + 1 of the lane 8
  // below: row shifts by 8 whose bank masks (banks are lane bits 3:2) write
  // only the receiving lanes.
#pragma unroll
  for (int j = 0; j < 8; j += 2)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int ia = 4 * j + k, ib = 4 * (j + 1) + k;
      const uint32_t nb = static_cast<uint32_t>(
          __builtin_amdgcn_update_dpp(static_cast<int>(w[ib]), static_cast<int>(w[ia]), 0x108, 0xF, 0x3, false));
      const uint32_t na = static_cast<uint32_t>(
          __builtin_amdgcn_update_dpp(static_cast<int>(w[ia]), static_cast<int>(w[ib]), 0x118, 0xF, 0xC, false));
      w[ia] = na;
      w[ib] = nb;
    }
  // Lanes with bit 4 set trade their piece j for piece j + 2 of the lane 16 below.
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int j = (jj & 1) | ((jj & 2) << 1);  // 0, 1, 4, 5
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const auto r = __builtin_amdgcn_permlane16_swap(w[4 * j + k], w[4 * (j + 2) + k], false, false);
      w[4 * j + k] = r[0];
      w[4 * (j + 2) + k] = r[1];
    }
  }
  // Lanes of the upper half trade their piece j for piece j + 4 of the lane 32 below.
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const auto r = __builtin_amdgcn_permlane32_swap(w[4 * j + k], w[4 * (j + 4) + k], false, false);
      w[4 * j + k] = r[0];
      w[4 * (j + 4) + k] = r[1];
    }
  uint8_t* base = chunk0 + static_cast<int64_t>(lane & 7) * chunk + off + 16 * (lane >> 3);
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    if (!(m < 4 ? valid_lo : valid_hi)) continue;
    *reinterpret_cast<uint4*>(base + 8 * m * chunk) = make_uint4(w[4 * m], w[4 * m + 1], w[4 * m + 2], w[4 * m + 3]);
  }
}

// kFromRam: expert e's record is stg row src_row[e] + base and the scale
// rows are copied; otherwise staging row j (a separate instantiation, so the
// staging path's code is not touched by the RAM-tier one).
template <int F, bool kFromRam>
__global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8, 8))) decode_kernel(DecodeArgs a) {
  __shared__ uint16_t s_lut[XP_LUT_BYTES + 32];  // the LUT, then the 64-byte position table
  __shared__ uint32_t s_ring[kGroupsPerBlock][kRingPad];

  const int j = blockIdx.x / a.blocks_per_row;
  int r = blockIdx.x % a.blocks_per_row;
  const int name = r < a.names[0].blocks ? 0 : 1;
  if (name == 1) r -= a.names[0].blocks;
  const NameDev nm = a.names[name];

  // Which expert, and whether it needs expanding (codec.py:263-277).
  const int64_t e = a.todo[j];
  bool active = e >= 0 && e < a.E;
  if (active && a.skip)
    for (int k = 0; k < a.K; ++k) active = active && a.skip[k] != e;
  if (!active || a.cache_row[e] >= 0) return;
  // A destination or record row outside its tensor is skipped, never clamped.
  const int64_t drow = a.dst_row[e];
  const int64_t srow = kFromRam ? a.src_row[e] + a.base : j;
  if (drow < 0 || drow >= nm.dst_rows || srow < 0 || srow >= nm.stg_rows) return;

  const int tid = threadIdx.x;
  // Read from the RAM tier, a launch that expands a single row is bound by
  // the latency of its loads over the host link, so both nibble words of an
  // iteration are fetched an iteration ahead; with more rows the link's
  // bandwidth is the bound, and the second word fetched at its iteration
  // paces the requests (fetching both early made 2-8 rows 13-20% slower).
  // The count looks at the first 256 entries of todo at most.
  bool early = false;
  if constexpr (kFromRam) {
    int rows = 0;
    const int scan = a.K < 256 ? a.K : 256;
    for (int k = 0; k < scan && rows < 2; ++k) {
      const int64_t ek = a.todo[k];
      rows += ek >= 0 && ek < a.E && a.cache_row[ek] < 0;
    }
    early = rows <= 1 && a.K <= 256;
  }
  // Read from the RAM tier, the name's first workgroup of the row also
  // copies the expert's scale row, which a staging gather would have moved.
  if constexpr (kFromRam) {
    if (r == 0)
      for (int i = tid; i < nm.scale_words; i += kThreads)
        nm.scale_dst[drow * nm.scale_words + i] = nm.scale[e * nm.scale_words + i];
  }
  const uint8_t* lut = a.lut + (e * a.num_names + name) * XP_LUT_BYTES;
  // The row's 9-bit table (entry = symbol << 4 | length) as length |
  // (exponent field << 3) << 8. Lengths are clamped to [1, LIMIT], which
  // leaves a valid table as it is and keeps the refill bound (and so every
  // ring read in range) for any table.
  if (tid < 64)
    reinterpret_cast<uint8_t*>(s_lut)[2 * XP_LUT_BYTES + tid] = static_cast<uint8_t>(tid > 63 - kLimit ? tid - 32 : tid);
  for (int i = tid; i < XP_LUT_BYTES; i += kThreads) {
    const uint32_t ent = lut[i];
    const uint32_t len = min(max(ent & 15u, 1u), static_cast<uint32_t>(kLimit));
    s_lut[i] = static_cast<uint16_t>(len | (((ent >> 4) << 3) << 8));
  }

  const int wave = tid >> 6, lane = tid & 63;
  const bool upper = lane >= 32;
  const uint32_t li = lane & 31;
  const uint32_t half_shift = upper ? 16u : 0u;
  const int G = nm.G;
  const int msteps = a.chunk / 8;
  const uint32_t* rec = reinterpret_cast<const uint32_t*>(nm.stg + srow * nm.pitch);
  const int64_t huff_off = (G + 1) + nm.N / 8;  // in words
  const int64_t maxw = nm.pitch / 4 - huff_off;

  const int gl = 2 * wave + (upper ? 1 : 0);  // the lane's group in the workgroup
  int g = r * kGroupsPerBlock + gl;
  const bool valid = g < G;
  if (!valid) g = G - 1;  // a spare half-wave repeats the last group and stores nothing
  int64_t gs = 0, ge = 0;
  if (maxw > 0) {
    gs = rec[g];
    ge = rec[g + 1];
    gs = gs < 0 ? 0 : (gs > maxw ? maxw : gs);
    ge = ge < gs ? gs : (ge > maxw ? maxw : ge);
  }
  Chain ch;
  // Words of the group, clamped as the ring state needs (no group consumes 65535).
  const uint32_t count = static_cast<uint32_t>(ge - gs < 0xFFFF ? ge - gs : 0xFFFF);
  // The record as a raw buffer of pitch bytes (stride 0; word 3 of the
  // descriptor 0x00020000 selects 32-bit data on gfx9-family chips): the
  // hardware range check returns zero for loads beyond it, so the group's
  // word and nibble loads need no clamps.
  const __amdgpu_buffer_rsrc_t rrec = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(rec), 0, static_cast<int>(nm.pitch), 0x00020000);
  ch.wsrc = static_cast<uint32_t>(4 * (huff_off + gs) + 4 * li);
  ch.ring = s_ring[gl];
  const uint32_t ring_addr = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ch.ring));
  ch.nib = static_cast<uint32_t>(4 * ((G + 1) + (int64_t(g) * msteps) * 32 + li));
  ch.buf = 0;
  ch.pos = 63u;  // nothing loaded: the first symbol refills every lane
  ch.b_val0 = ch.b_val1 = 0;
  uint8_t* out = nm.dst + drow * nm.N + int64_t(g) * 32 * a.chunk;  // chunk 0 of the group
  // The wave's two groups as one run of 64 chunks (the 16-iteration flush).
  const int g_lo = r * kGroupsPerBlock + 2 * __builtin_amdgcn_readfirstlane(wave);
  uint8_t* out_wave = nm.dst + drow * nm.N + int64_t(g_lo) * 32 * a.chunk;
  const bool valid_lo = g_lo < G, valid_hi = g_lo + 1 < G;
  // Initial fill of the ring: the group's first kRing words (8 loads per lane).
  {
    uint32_t v[kRing / 32];
#pragma unroll
    for (uint32_t i = 0; i < kRing / 32; ++i) {
      v[i] = __builtin_amdgcn_raw_buffer_load_b32(rrec, ch.wsrc + 128u * i, 0, 0);
    }
#pragma unroll
    for (uint32_t i = 0; i < kRing / 32; ++i) {
      const uint32_t w = li + 32 * i;
      ch.ring[w] = v[i];
      if (w < kMirror) ch.ring[w + kRing] = v[i];
    }
    ch.x_next = __builtin_amdgcn_raw_buffer_load_b32(rrec, ch.nib, 0, 0);
    ch.x_next1 = early ? __builtin_amdgcn_raw_buffer_load_b32(rrec, ch.nib, 128, 0) : 0u;
  }
  Rings rg;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    rg.count[h] = __builtin_amdgcn_readlane(count, 32 * h);
    rg.base[h] = __builtin_amdgcn_readlane(ring_addr, 32 * h) >> 2;
    rg.rp[h] = rg.bb[h] = rg.bn[h] = 0;
    rg.fe[h] = rg.q[h] = rg.count[h] < kRing ? rg.count[h] : kRing;
    rg.ab0[h] = rg.base[h];
  }
  __syncthreads();

  // Output: a lane's chunk is contiguous, produced 8 bytes per iteration.
  // F iterations (8F bytes) are gathered in registers and stored together
  // (see flush): lines written in 16-byte pieces far apart in time leave the
  // caches as partial writes, which cost more than the decode itself.
  // The main loop, instantiated for each nibble fetch policy (a branch
  // inside it changed how the compiler scheduled the loads of the other).
  auto run = [&](auto early_c) __attribute__((always_inline)) {
    constexpr bool kEarly = decltype(early_c)::value;
    uint4 ob[F / 2];
#pragma unroll
    for (int i = 0; i < F / 2; ++i) ob[i] = make_uint4(0, 0, 0, 0);
    for (int m0 = 0; m0 < msteps; m0 += F) {
      // Priority by progress through the chunk: the first workgroups of a
      // 256-row launch otherwise took 78 against 116 us for those dispatched
      // a microsecond later, and the launch 3% longer; a 64-row launch 10%.
      progress_priority(m0, msteps);
#pragma unroll
      for (int u = 0; u < F; u += 2) {
        const int m = m0 + u;
        const uint32_t x0 = ch.x_next;
        uint32_t x1;
        if constexpr (kEarly) {
          x1 = ch.x_next1;
          ch.x_next1 = __builtin_amdgcn_raw_buffer_load_b32(rrec, ch.nib, 128 * (m + 3 < msteps ? m + 3 : m + 1), 0);
        } else {
          x1 = __builtin_amdgcn_raw_buffer_load_b32(rrec, ch.nib, 128 * (m + 1), 0);
        }
        ch.x_next = __builtin_amdgcn_raw_buffer_load_b32(rrec, ch.nib, 128 * (m + 2 < msteps ? m + 2 : m), 0);
        uint2 o0 = nibble_template(x0), o1 = nibble_template(x1);
        half_begin(rg, ch, li, upper, half_shift, rrec);
        // The next unread ring word of each half's group, packed in a scalar register.
        uint32_t offs = spack(rg.ab0[0], rg.ab0[1]);
        __builtin_amdgcn_wave_barrier();
        o0.x = quad(ch, offs, half_shift, s_lut, o0.x);
        o0.y = quad(ch, offs, half_shift, s_lut, o0.y);
        o1.x = quad(ch, offs, half_shift, s_lut, o1.x);
        o1.y = quad(ch, offs, half_shift, s_lut, o1.y);
        __builtin_amdgcn_wave_barrier();
        half_end(rg, ch, li, half_shift, offs);
        ob[u >> 1] = make_uint4(o0.x, o0.y, o1.x, o1.y);
      }
      if constexpr (F == 16)
        flush16(ob, out_wave, a.chunk, static_cast<uint32_t>(lane), 8 * m0, valid_lo, valid_hi);
      else
        flush<F>(ob, out, a.chunk, li, 8 * m0, valid);
    }
  };
  if (kFromRam && early)
    run(std::true_type{});
  else
    run(std::false_type{});
}

}  // namespace
}  // namespace xp

using namespace xp;

namespace {

// Shared by both decode entry points: src_row == nullptr reads staging row j
// (no scales), else RAM-tier row src_row[e] + base and copies the scales.
int launch_decode(const char* what, const int64_t* todo, int64_t K, int64_t num_experts, const int64_t* dst_row,
                  const int64_t* cache_row, const int64_t* src_row, int64_t base, const uint8_t* lut,
                  const xp_decode_name* names, int num_names, const xp_decode_scale* scales, const int64_t* skip,
                  int64_t chunk, void* stream) {
  XP_REQUIRE(K >= 0 && K <= (1 << 20), "%s: K=%lld", what, (long long)K);
  XP_REQUIRE(num_names >= 1 && num_names <= 2 && names, "%s: %d names (1 or 2)", what, num_names);
  XP_REQUIRE(chunk >= 32 && chunk % 32 == 0 && chunk <= 4096, "%s: chunk=%lld (multiple of 32)", what,
             (long long)chunk);
  XP_REQUIRE(num_experts >= 1, "%s: num_experts=%lld", what, (long long)num_experts);
  if (K == 0) return XP_OK;
  XP_REQUIRE(todo && dst_row && cache_row && lut, "%s: null index tensor", what);
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
  a.src_row = src_row;
  a.base = base;
  int per_row = 0;
  for (int n = 0; n < num_names; ++n) {
    const xp_decode_name& s = names[n];
    const int64_t group = chunk * XP_LANES;
    XP_REQUIRE(s.row_bytes > 0 && s.row_bytes % group == 0, "%s: name %d row of %lld values is not a multiple of %lld",
               what, n, (long long)s.row_bytes, (long long)group);
    const int64_t G = s.row_bytes / group;
    XP_REQUIRE(s.pitch < (int64_t(1) << 31), "%s: name %d pitch %lld is 2 GiB or more", what, n, (long long)s.pitch);
    XP_REQUIRE(s.pitch % 4 == 0 && s.pitch >= 4 * (G + 1) + s.row_bytes / 2,
               "%s: name %d pitch %lld cannot hold the record header", what, n, (long long)s.pitch);
    XP_REQUIRE(s.stg && s.dst, "%s: name %d has a null buffer", what, n);
    XP_REQUIRE(aligned16(s.stg) && aligned16(s.dst) && s.pitch % 16 == 0,
               "%s: name %d buffers and pitch must be 16-byte aligned", what, n);
    a.names[n] = NameDev{static_cast<const uint8_t*>(s.stg),
                         s.pitch,
                         s.stg_rows,
                         static_cast<uint8_t*>(s.dst),
                         s.dst_rows,
                         s.row_bytes,
                         static_cast<int>(G),
                         static_cast<int>((G + kGroupsPerBlock - 1) / kGroupsPerBlock),
                         nullptr,
                         nullptr,
                         0};
    if (scales) {
      const xp_decode_scale& c = scales[n];
      XP_REQUIRE(c.scale && c.scale_dst, "%s: name %d has a null scale buffer", what, n);
      XP_REQUIRE(c.scale_bytes > 0 && c.scale_bytes % 4 == 0 && c.scale_bytes < (int64_t(1) << 20),
                 "%s: name %d scale rows of %lld bytes (a positive multiple of 4 below 1 MiB)", what, n,
                 (long long)c.scale_bytes);
      XP_REQUIRE(c.scale_rows >= num_experts && c.scale_dst_rows >= s.dst_rows,
                 "%s: name %d scale rows %lld / %lld, need %lld experts and %lld destination rows", what, n,
                 (long long)c.scale_rows, (long long)c.scale_dst_rows, (long long)num_experts,
                 (long long)s.dst_rows);
      XP_REQUIRE(aligned4(c.scale) && aligned4(c.scale_dst), "%s: name %d scale buffers must be 4-byte aligned",
                 what, n);
      a.names[n].scale = static_cast<const uint32_t*>(c.scale);
      a.names[n].scale_dst = static_cast<uint32_t*>(c.scale_dst);
      a.names[n].scale_words = static_cast<int>(c.scale_bytes / 4);
    }
    per_row += a.names[n].blocks;
  }
  if (num_names == 1) a.names[1] = a.names[0];
  a.blocks_per_row = per_row;
  const int64_t grid = K * per_row;
  XP_REQUIRE(grid <= (int64_t(1) << 31) - 1, "%s: grid too large", what);
  // Runs of 128 bytes per store (8-lane sets) when the chunk allows it, else 64 or 32.
  const dim3 g(static_cast<unsigned>(grid)), b(kThreads);
  if (src_row) {
    if (chunk % 128 == 0)
      hipLaunchKernelGGL((decode_kernel<16, true>), g, b, 0, as_stream(stream), a);
    else if (chunk % 64 == 0)
      hipLaunchKernelGGL((decode_kernel<8, true>), g, b, 0, as_stream(stream), a);
    else
      hipLaunchKernelGGL((decode_kernel<4, true>), g, b, 0, as_stream(stream), a);
  } else if (chunk % 128 == 0) {
    hipLaunchKernelGGL((decode_kernel<16, false>), g, b, 0, as_stream(stream), a);
  } else if (chunk % 64 == 0) {
    hipLaunchKernelGGL((decode_kernel<8, false>), g, b, 0, as_stream(stream), a);
  } else {
    hipLaunchKernelGGL((decode_kernel<4, false>), g, b, 0, as_stream(stream), a);
  }
  return check_launch("decode_kernel");
}

}  // namespace

extern "C" {

int xp_decode_rows(const int64_t* todo, int64_t K, int64_t num_experts, const int64_t* dst_row,
                   const int64_t* cache_row, const uint8_t* lut, const xp_decode_name* names, int num_names,
                   const int64_t* skip, int64_t chunk, void* stream) {
  return launch_decode("xp_decode_rows", todo, K, num_experts, dst_row, cache_row, nullptr, 0, lut, names, num_names,
                       nullptr, skip, chunk, stream);
}

int xp_decode_rows_from_ram(const int64_t* todo, int64_t K, int64_t num_experts, const int64_t* dst_row,
                            const int64_t* cache_row, const int64_t* src_row, int64_t base, const uint8_t* lut,
                            const xp_decode_name* names, int num_names, const xp_decode_scale* scales,
                            const int64_t* skip, int64_t chunk, void* stream) {
  XP_REQUIRE(src_row && scales, "xp_decode_rows_from_ram: src_row and scales must be non-null");
  return launch_decode("xp_decode_rows_from_ram", todo, K, num_experts, dst_row, cache_row, src_row, base, lut, names,
                       num_names, scales, skip, chunk, stream);
}

}  // extern "C"
