// Zstandard frame decoding (RFC 8878), written once for a team of lanes that
// run it together: a 64-lane workgroup on the GPU (zstd_decode.hip). The
// frame, block and section headers are parsed by every lane alike (the same
// bytes, the same branches); table construction and the Huffman streams run
// on single lanes with the tables in shared memory; literal and match copies
// are spread over all lanes.
//
// A Team provides lane() (0 .. size-1), size and sync() (a barrier that also
// makes every lane's earlier global and shared-memory writes visible to the
// team).
//
// Every read of the input is bounds-checked; malformed input ends the task
// with an error code, never with an out-of-bounds access. Not supported:
// dictionaries (a frame naming a dictionary is an error) and checking the
// optional content checksum (its 4 bytes are skipped).
#pragma once

#include <stdint.h>

namespace bs_zstd {

constexpr uint32_t kBlockMax = 128u << 10;     // RFC 8878 3.1.1.2.4: Block_Maximum_Size
constexpr uint32_t kHufLogMax = 12;
constexpr uint32_t kLLLog = 9, kMLLog = 9, kOFLog = 8, kWeightLog = 6;
constexpr uint32_t kLLMax = 35, kMLMax = 52, kOFMax = 31;
constexpr uint32_t kStageBytes = 24u << 10;    // compressed blocks up to this size are read from shared memory

enum : int32_t {
  kOk = 0,
  kErrTruncated = 1,     // a header or section runs past the input
  kErrFormat = 2,        // bad magic, reserved bits or block type, dictionary frame
  kErrTable = 3,         // invalid FSE or Huffman table description
  kErrStream = 4,        // a bitstream does not end where it must
  kErrOutput = 5,        // output past the destination capacity, or a size check failed
  kErrOffset = 6,        // a match reaches before the start of its frame
};

struct FseCell {
  uint16_t base;     // next state = base + (nb bits read)
  uint8_t sym;
  uint8_t nb;
};

// Per-task state: the decode tables kept between the blocks of a frame.
struct ZState {
  uint16_t huf[1u << kHufLogMax];     // symbol | bits << 8, indexed by the next huf_log bits
  FseCell ll[1u << kLLLog], ml[1u << kMLLog], of[1u << kOFLog];
  FseCell wt[1u << kWeightLog];       // Huffman-weight table
  uint32_t ll_base[kLLMax + 1], ml_base[kMLMax + 1];
  uint8_t ll_bits[kLLMax + 1], ml_bits[kMLMax + 1];
  int16_t norm[64];
  uint16_t next[64];                  // FSE construction: next state per symbol
  uint8_t weight[256];
  uint32_t huf_log;                   // 0: no Huffman table yet in this frame
  uint32_t ll_log, ml_log, of_log;
  uint32_t have_ll, have_ml, have_of; // a table exists for the Repeat mode
  uint32_t seq_pos;                   // broadcast: where the sequence bitstream starts
  int32_t err;                        // broadcast: error of single-lane work
  uint8_t stage[kStageBytes];         // the current compressed block, when it fits
};

__host__ __device__ __forceinline__ uint32_t highbit(uint32_t v) { return 31u - (uint32_t)__builtin_clz(v); }
__host__ __device__ __forceinline__ uint64_t mask64(uint32_t n) { return n >= 64 ? ~0ull : ((1ull << n) - 1ull); }

// Little-endian value of p[i .. i+8), bytes at or past `len` read as zero.
__host__ __device__ inline uint64_t load_le(const uint8_t* p, uint64_t len, uint64_t i) {
  uint64_t v = 0;
  for (uint32_t k = 0; k < 8; ++k)
    if (i + k < len) v |= (uint64_t)p[i + k] << (8 * k);
  return v;
}

// Forward bit reader (FSE table descriptions): bits taken from the least
// significant end of each byte, bytes in increasing order.
struct FwdBits {
  const uint8_t* p;
  uint64_t len;
  uint64_t pos;      // bits consumed
  __host__ __device__ uint32_t peek(uint32_t n) const {
    return (uint32_t)((load_le(p, len, pos >> 3) >> (pos & 7)) & mask64(n));
  }
  __host__ __device__ uint32_t read(uint32_t n) {
    const uint32_t v = peek(n);
    pos += n;
    return v;
  }
};

// Backward bit reader (Huffman and FSE-coded streams, RFC 8878 4.1, 4.2.2):
// the stream is read from its last byte towards its first; the highest set
// bit of the last byte marks the end and is skipped. Reading n bits yields the
// next n unread bits from the top as one number; past the start of the stream
// the missing bits read as zeros and `bits` goes negative (overflow). The next
// unread bits sit left-aligned in a 64-bit register, refilled a byte at a time.
struct BackBits {
  const uint8_t* p;
  uint64_t acc;      // the top `have` unread bits, most significant first; zeros below
  int32_t have;      // negative once reads have gone past the start of the stream
  uint32_t lo;       // bytes [0, lo) are not yet in acc
  __host__ __device__ bool init(const uint8_t* q, uint64_t n) {
    p = q;
    acc = 0;
    have = 0;
    lo = 0;
    if (n == 0 || n > 0xFFFFFFFFull || q[n - 1] == 0) return false;
    const uint32_t hb = highbit(q[n - 1]);
    acc = hb ? (uint64_t)(q[n - 1] & ((1u << hb) - 1u)) << (64 - hb) : 0ull;
    have = (int32_t)hb;
    lo = (uint32_t)(n - 1);
    refill();
    return true;
  }
  // Unread bits; negative after an overflow.
  __host__ __device__ int64_t bits() const { return (int64_t)lo * 8 + have; }
  __host__ __device__ void refill() {         // as many whole bytes as fit, loaded together
    if (have > 56 || lo == 0) return;
    const uint32_t want = (uint32_t)(64 - have) >> 3;
    const uint32_t k = lo < want ? lo : want;
    uint64_t v = 0;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i)
      if (i < k) v |= (uint64_t)p[lo - 1 - i] << (56 - 8 * i);
    acc |= v >> have;
    have += (int32_t)(8 * k);
    lo -= k;
  }
  __host__ __device__ uint32_t peek(uint32_t n) {             // n <= 32
    if (have < (int32_t)n) refill();
    return n ? (uint32_t)(acc >> (64 - n)) : 0u;
  }
  __host__ __device__ void skip(uint32_t n) {                 // after a peek of >= n bits
    acc = n < 64 ? acc << n : 0ull;
    have -= (int32_t)n;
  }
  __host__ __device__ uint32_t read(uint32_t n) {
    const uint32_t v = peek(n);
    skip(n);
    return v;
  }
};

// Default distributions (RFC 8878 3.1.1.3.2.2), 3 bits per symbol holding
// count + 1, 21 symbols per word.
__host__ __device__ inline int16_t default_norm(uint32_t kind, uint32_t s) {
  uint64_t w;
  const uint32_t k = s / 21, sh = 3 * (s % 21);
  if (kind == 0)
    w = k == 0 ? 0x36DB4936DB6DB6E5ull : 0x000000009249C6DBull;                  // literal lengths, 36
  else if (kind == 1)
    w = k == 0 ? 0x24924924936DB72Aull : k == 1 ? 0x2492492492492492ull : 0x0000000000000492ull;  // match lengths, 53
  else
    w = k == 0 ? 0x24924924936D2492ull : 0x0000000000000092ull;                  // offsets, 29
  return (int16_t)((w >> sh) & 7u) - 1;
}

// Extra-bit counts of the literal- and match-length codes (RFC 8878
// 3.1.1.3.2.1.1); each baseline is the previous one plus 2^(previous bits).
__host__ __device__ inline uint32_t ll_code_bits(uint32_t c) {
  return c < 16 ? 0u : c < 20 ? 1u : c < 22 ? 2u : c < 24 ? 3u : c == 24 ? 4u : c - 19u;
}
__host__ __device__ inline uint32_t ml_code_bits(uint32_t c) {
  return c < 32 ? 0u : c < 36 ? 1u : c < 38 ? 2u : c < 40 ? 3u : c < 42 ? 4u : c == 42 ? 5u : c - 36u;
}
__host__ __device__ inline void build_length_codes(ZState& z) {
  uint32_t b = 0;
  for (uint32_t c = 0; c <= kLLMax; ++c) {
    z.ll_bits[c] = (uint8_t)ll_code_bits(c);
    z.ll_base[c] = c < 16 ? c : b;
    b = (c < 16 ? c : b) + (1u << ll_code_bits(c));
  }
  b = 0;
  for (uint32_t c = 0; c <= kMLMax; ++c) {
    z.ml_bits[c] = (uint8_t)ml_code_bits(c);
    z.ml_base[c] = c < 32 ? c + 3 : b;
    b = (c < 32 ? c + 3 : b) + (1u << ml_code_bits(c));
  }
}

// FSE table description (RFC 8878 4.1.1) at p[0, len) into norm[]; returns
// the bytes it takes, 0 if it is invalid.
__host__ __device__ inline uint32_t read_ncount(const uint8_t* p, uint64_t len, int16_t* norm, uint32_t max_sym,
                                                uint32_t max_log, uint32_t& log, uint32_t& nsym) {
  if (len == 0) return 0;
  FwdBits br{p, len, 0};
  log = br.read(4) + 5;
  if (log > max_log) return 0;
  int32_t remaining = (1 << log) + 1, threshold = 1 << log;
  uint32_t nb = log + 1, sym = 0;
  bool prev0 = false;
  while (remaining > 1 && sym <= max_sym) {
    if (prev0) {                        // a zero count is followed by 2-bit repeat flags
      uint32_t n0 = sym;
      for (;;) {
        const uint32_t r = br.read(2);
        n0 += r;
        if (r != 3 || n0 > max_sym) break;
      }
      if (n0 > max_sym) return 0;
      while (sym < n0) norm[sym++] = 0;
    }
    const int32_t maxv = (2 * threshold - 1) - remaining;
    const uint32_t v = br.peek(nb);
    int32_t count;
    if ((int32_t)(v & (uint32_t)(threshold - 1)) < maxv) {
      count = (int32_t)(v & (uint32_t)(threshold - 1));
      br.pos += nb - 1;
    } else {
      count = (int32_t)(v & (uint32_t)(2 * threshold - 1));
      if (count >= threshold) count -= maxv;
      br.pos += nb;
    }
    --count;                            // -1: a "less than one" probability
    remaining -= count < 0 ? -count : count;
    norm[sym++] = (int16_t)count;
    prev0 = count == 0;
    while (remaining < threshold) {
      --nb;
      threshold >>= 1;
    }
  }
  if (remaining != 1 || br.pos > 8 * len) return 0;
  nsym = sym;
  return (uint32_t)((br.pos + 7) >> 3);
}

// Decode table for norm[0, nsym) at accuracy `log` (RFC 8878 4.1.1, "FSE
// Table Construction"). False if the counts do not fill the table.
__host__ __device__ inline bool build_fse(FseCell* t, const int16_t* norm, uint32_t nsym, uint32_t log,
                                          uint16_t* next) {
  const uint32_t size = 1u << log, mask = size - 1;
  uint32_t high = size - 1;
  uint32_t total = 0;
  if (nsym > 64) return false;
  for (uint32_t s = 0; s < nsym; ++s) {
    if (norm[s] == -1) {
      t[high--].sym = (uint8_t)s;
      next[s] = 1;
      ++total;
    } else {
      next[s] = (uint16_t)(norm[s] < 0 ? 0 : norm[s]);
      total += next[s];
    }
  }
  if (total != size) return false;
  const uint32_t step = (size >> 1) + (size >> 3) + 3;
  uint32_t pos = 0;
  for (uint32_t s = 0; s < nsym; ++s)
    for (int32_t i = 0; i < norm[s]; ++i) {
      t[pos].sym = (uint8_t)s;
      do pos = (pos + step) & mask;
      while (pos > high);
    }
  if (pos != 0) return false;
  for (uint32_t u = 0; u < size; ++u) {
    const uint32_t x = next[t[u].sym]++;
    const uint32_t nb = log - highbit(x);
    t[u].nb = (uint8_t)nb;
    t[u].base = (uint16_t)((x << nb) - size);
  }
  return true;
}

// Size in bytes of a Huffman tree description starting at q (RFC 8878 4.2.1).
__host__ __device__ inline uint32_t huf_desc_bytes(uint8_t h) { return h < 128 ? 1u + h : 1u + (h - 127u + 1u) / 2u; }

// Builds z.huf from the tree description at q[0, n) (n >= its size): the
// weights, the implied last weight, then codes assigned by weight and symbol.
__host__ __device__ inline int32_t build_huffman(ZState& z, const uint8_t* q, uint64_t n) {
  const uint8_t h = q[0];
  uint32_t nw = 0;
  if (h >= 128) {
    nw = h - 127u;
    for (uint32_t i = 0; i < nw; ++i) {
      const uint8_t b = q[1 + i / 2];
      z.weight[i] = (uint8_t)((i & 1) ? (b & 15u) : (b >> 4));
    }
  } else {
    uint32_t log = 0, nsym = 0;
    const uint32_t used = read_ncount(q + 1, h, z.norm, kHufLogMax, kWeightLog, log, nsym);
    if (!used || !build_fse(z.wt, z.norm, nsym, log, z.next)) return kErrTable;
    BackBits br;
    if (used >= h || !br.init(q + 1 + used, h - used)) return kErrTable;
    uint32_t s1 = br.read(log), s2 = br.read(log);
    for (;;) {                          // two interleaved states until the stream overflows
      if (nw >= 255) return kErrTable;
      z.weight[nw++] = z.wt[s1].sym;
      s1 = z.wt[s1].base + br.read(z.wt[s1].nb);
      if (br.bits() < 0) {
        z.weight[nw++] = z.wt[s2].sym;
        break;
      }
      if (nw >= 255) return kErrTable;
      z.weight[nw++] = z.wt[s2].sym;
      s2 = z.wt[s2].base + br.read(z.wt[s2].nb);
      if (br.bits() < 0) {
        z.weight[nw++] = z.wt[s1].sym;
        break;
      }
    }
    if (nw > 255) return kErrTable;
  }
  (void)n;
  uint32_t total = 0;
  for (uint32_t i = 0; i < nw; ++i) {
    if (z.weight[i] > kHufLogMax) return kErrTable;
    if (z.weight[i]) total += 1u << (z.weight[i] - 1);
  }
  if (total == 0) return kErrTable;
  const uint32_t log = highbit(total) + 1;
  if (log > kHufLogMax) return kErrTable;
  const uint32_t rest = (1u << log) - total;
  if (rest & (rest - 1)) return kErrTable;
  z.weight[nw] = (uint8_t)(highbit(rest) + 1);
  const uint32_t nsym = nw + 1;
  uint32_t pos = 0;
  for (uint32_t w = 1; w <= log; ++w)
    for (uint32_t s = 0; s < nsym; ++s)
      if (z.weight[s] == w) {
        const uint16_t e = (uint16_t)(s | ((log + 1 - w) << 8));
        for (uint32_t k = 0; k < (1u << (w - 1)); ++k) z.huf[pos++] = e;
      }
  if (pos != (1u << log)) return kErrTable;
  z.huf_log = log;
  return kOk;
}

// One Huffman-coded literal stream into out[0, count).
__host__ __device__ inline bool huf_stream(const ZState& z, const uint8_t* s, uint64_t n, uint8_t* out,
                                           uint32_t count) {
  BackBits br;
  if (!br.init(s, n)) return false;
  const uint32_t log = z.huf_log;
  uint32_t k = 0;
  // four symbols per refill while at least 4 * log bits are loaded (log <= 12)
  for (; k + 4 <= count; k += 4) {
    br.refill();
    if (br.have < (int32_t)(4 * log)) break;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint16_t e = z.huf[br.acc >> (64 - log)];
      out[k + j] = (uint8_t)e;
      br.skip(e >> 8);
    }
  }
  for (; k < count; ++k) {
    const uint16_t e = z.huf[br.peek(log)];
    out[k] = (uint8_t)e;
    br.skip(e >> 8);
  }
  return br.bits() == 0;
}

// Sets up one sequence table (literal lengths 0, offsets 1, match lengths 2)
// for `mode` from b[pos ...]; returns the bytes taken or -1.
__host__ __device__ inline int32_t seq_table(ZState& z, uint32_t kind, uint32_t mode, const uint8_t* b, uint64_t n) {
  FseCell* t = kind == 0 ? z.ll : kind == 1 ? z.of : z.ml;
  uint32_t* log = kind == 0 ? &z.ll_log : kind == 1 ? &z.of_log : &z.ml_log;
  uint32_t* have = kind == 0 ? &z.have_ll : kind == 1 ? &z.have_of : &z.have_ml;
  const uint32_t max_sym = kind == 0 ? kLLMax : kind == 1 ? kOFMax : kMLMax;
  const uint32_t max_log = kind == 0 ? kLLLog : kind == 1 ? kOFLog : kMLLog;
  if (mode == 0) {                      // predefined
    const uint32_t dkind = kind == 0 ? 0u : kind == 1 ? 2u : 1u;
    const uint32_t nsym = kind == 0 ? 36u : kind == 1 ? 29u : 53u;
    for (uint32_t s = 0; s < nsym; ++s) z.norm[s] = default_norm(dkind, s);
    *log = kind == 1 ? 5u : 6u;
    if (!build_fse(t, z.norm, nsym, *log, z.next)) return -1;
    *have = 1;
    return 0;
  }
  if (mode == 1) {                      // RLE: one symbol
    if (n < 1 || b[0] > max_sym) return -1;
    t[0] = FseCell{0, b[0], 0};
    *log = 0;
    *have = 1;
    return 1;
  }
  if (mode == 2) {                      // FSE-compressed
    uint32_t lg = 0, nsym = 0;
    const uint32_t used = read_ncount(b, n, z.norm, max_sym, max_log, lg, nsym);
    if (!used || !build_fse(t, z.norm, nsym, lg, z.next)) return -1;
    *log = lg;
    *have = 1;
    return (int32_t)used;
  }
  return *have ? 0 : -1;                // repeat
}

// Repeat offsets (RFC 8878 3.1.2.5), kept from block to block in a frame.
struct Rep {
  uint32_t r0, r1, r2;
};

// Output positions are frame-relative inside dst; `frame0` is where the frame
// starts. Every lane holds the same values.
struct Out {
  uint8_t* dst;
  uint64_t cap;
  uint64_t op;
  uint64_t frame0;
};

template <class Team>
__host__ __device__ inline void team_fill(const Team& tm, uint8_t* d, uint8_t v, uint64_t n) {
  for (uint64_t i = tm.lane(); i < n; i += Team::size) d[i] = v;
}
template <class Team>
__host__ __device__ inline void team_copy(const Team& tm, uint8_t* d, const uint8_t* s, uint64_t n) {
  for (uint64_t i = tm.lane(); i < n; i += Team::size) d[i] = s[i];
}

// One compressed block b[0, n) (RFC 8878 3.1.1.3). rep: repeat offsets.
template <class Team>
__host__ __device__ __forceinline__ int32_t zstd_block(const Team& tm, ZState& z, const uint8_t* b, uint64_t n,
                                                       Out& o, Rep& rep, uint8_t* lit_buf) {
  if (n < 1) return kErrTruncated;
  const uint32_t ltype = b[0] & 3u, sf = (b[0] >> 2) & 3u;
  uint32_t lh, lsize, lcsize = 0;
  bool four = false;
  if (ltype < 2) {
    lh = (sf & 1u) ? (sf == 1 ? 2u : 3u) : 1u;
    if (n < lh) return kErrTruncated;
    const uint32_t v = (uint32_t)load_le(b, lh, 0);
    lsize = lh == 1 ? v >> 3 : v >> 4;
  } else {
    lh = sf < 2 ? 3u : sf == 2 ? 4u : 5u;
    if (n < lh) return kErrTruncated;
    const uint64_t v = load_le(b, lh, 0);
    four = sf != 0;
    if (sf < 2) {
      lsize = (uint32_t)(v >> 4) & 0x3FFu;
      lcsize = (uint32_t)(v >> 14) & 0x3FFu;
    } else if (sf == 2) {
      lsize = (uint32_t)(v >> 4) & 0x3FFFu;
      lcsize = (uint32_t)(v >> 18) & 0x3FFFu;
    } else {
      lsize = (uint32_t)(v >> 4) & 0x3FFFFu;
      lcsize = (uint32_t)(v >> 22) & 0x3FFFFu;
    }
  }
  if (lsize > kBlockMax) return kErrFormat;
  uint64_t pos = lh;
  const uint8_t* lit = lit_buf;
  if (ltype == 0) {                     // raw literals: read in place
    if (pos + lsize > n) return kErrTruncated;
    lit = b + pos;
    pos += lsize;
  } else if (ltype == 1) {              // RLE literals
    if (pos + 1 > n) return kErrTruncated;
    team_fill(tm, lit_buf, b[pos], lsize);
    tm.sync();
    pos += 1;
  } else {                              // Huffman-coded (2: with a new tree, 3: the previous tree)
    if (pos + lcsize > n) return kErrTruncated;
    const uint8_t* q = b + pos;
    uint32_t tree = 0;
    if (ltype == 2) {
      if (lcsize < 1) return kErrTruncated;
      tree = huf_desc_bytes(q[0]);
      if (tree > lcsize) return kErrTruncated;
      if (tm.lane() == 0) z.err = build_huffman(z, q, tree);
      tm.sync();
      const int32_t e = z.err;
      tm.sync();
      if (e) return e;
    } else if (z.huf_log == 0) {
      return kErrTable;
    }
    const uint8_t* s = q + tree;
    const uint32_t sn = lcsize - tree;
    if (!four) {
      if (tm.lane() == 0) z.err = huf_stream(z, s, sn, lit_buf, lsize) ? kOk : kErrStream;
    } else {
      if (sn < 6) return kErrTruncated;
      const uint32_t l1 = (uint32_t)load_le(s, 2, 0), l2 = (uint32_t)load_le(s + 2, 2, 0),
                     l3 = (uint32_t)load_le(s + 4, 2, 0);
      if (6ull + l1 + l2 + l3 > sn) return kErrTruncated;
      const uint32_t l4 = sn - 6 - l1 - l2 - l3;
      const uint32_t seg = (lsize + 3) / 4;
      if (3 * seg > lsize) return kErrFormat;
      if (tm.lane() == 0) z.err = kOk;
      tm.sync();
      const uint32_t k = tm.lane();
      for (uint32_t st = k; st < 4; st += Team::size) {
        const uint32_t off = 6 + (st > 0 ? l1 : 0) + (st > 1 ? l2 : 0) + (st > 2 ? l3 : 0);
        const uint32_t len = st == 0 ? l1 : st == 1 ? l2 : st == 2 ? l3 : l4;
        const uint32_t cnt = st < 3 ? seg : lsize - 3 * seg;
        if (!huf_stream(z, s + off, len, lit_buf + (uint64_t)st * seg, cnt)) z.err = kErrStream;
      }
    }
    tm.sync();
    const int32_t e = z.err;
    if (e) return e;
    pos += lcsize;
  }

  // sequences section header (RFC 8878 3.1.1.3.2.1)
  if (pos >= n) return kErrTruncated;
  uint32_t nseq = b[pos];
  if (nseq == 0) {
    pos += 1;
  } else if (nseq < 128) {
    pos += 1;
  } else if (nseq < 255) {
    if (pos + 2 > n) return kErrTruncated;
    nseq = ((nseq - 128) << 8) + b[pos + 1];
    pos += 2;
  } else {
    if (pos + 3 > n) return kErrTruncated;
    nseq = b[pos + 1] + ((uint32_t)b[pos + 2] << 8) + 0x7F00u;
    pos += 3;
  }
  uint64_t lp = 0;                      // literals consumed
  if (nseq > 0) {
    if (pos >= n) return kErrTruncated;
    const uint32_t modes = b[pos++];
    if (modes & 3u) return kErrFormat;
    tm.sync();                          // every lane has read z.err before lane 0 reuses it
    if (tm.lane() == 0) {
      int32_t e = kOk;
      uint64_t p = pos;
      for (uint32_t k = 0; k < 3 && e == kOk; ++k) {     // LL, OF, ML
        const uint32_t mode = (modes >> (6 - 2 * k)) & 3u;
        const int32_t used = seq_table(z, k, mode, b + p, n - p);
        if (used < 0) e = kErrTable;
        else p += (uint32_t)used;
      }
      z.err = e;
      z.seq_pos = (uint32_t)p;
    }
    tm.sync();
    if (z.err) return z.err;
    pos = z.seq_pos;
    BackBits br;
    if (pos >= n || !br.init(b + pos, n - pos)) return kErrStream;
    uint32_t sll = br.read(z.ll_log), sof = br.read(z.of_log), sml = br.read(z.ml_log);
    uint64_t visible = o.op;            // every lane's output below this is visible to all
    for (uint32_t i = 0; i < nseq; ++i) {
      const FseCell cl = z.ll[sll], co = z.of[sof], cm = z.ml[sml];
      if (co.sym > kOFMax) return kErrStream;
      const uint32_t ofv = (1u << co.sym) + br.read(co.sym);
      const uint32_t ml = z.ml_base[cm.sym] + br.read(z.ml_bits[cm.sym]);
      const uint32_t ll = z.ll_base[cl.sym] + br.read(z.ll_bits[cl.sym]);
      uint32_t off;
      if (ofv > 3) {
        off = ofv - 3;
        rep.r2 = rep.r1;
        rep.r1 = rep.r0;
        rep.r0 = off;
      } else {                          // a repeat: shifted by one when the literal length is 0
        const uint32_t r = ofv - 1 + (ll == 0 ? 1u : 0u);
        if (r == 0) {
          off = rep.r0;
        } else {
          off = r == 1 ? rep.r1 : r == 2 ? rep.r2 : rep.r0 - 1;
          if (r != 1) rep.r2 = rep.r1;
          rep.r1 = rep.r0;
          rep.r0 = off;
        }
      }
      if (i + 1 < nseq) {               // state updates: literal lengths, match lengths, offsets
        sll = cl.base + br.read(cl.nb);
        sml = cm.base + br.read(cm.nb);
        sof = co.base + br.read(co.nb);
      }
      if (br.bits() < 0) return kErrStream;
      if (lp + ll > lsize) return kErrStream;
      if (o.op + ll + ml > o.cap) return kErrOutput;
      if (off == 0 || off > o.op + ll - o.frame0) return kErrOffset;
      // match byte i is d[ll - off + i % off]: earlier output, or this
      // sequence's literals (then read from the literal buffer). Output below
      // `visible` has been written before the last barrier; a match that reads
      // above it waits for one first.
      const uint64_t from = o.op + ll - off;
      const uint64_t reach = from + (off < ml ? off : ml);
      if ((reach < o.op ? reach : o.op) > visible) {
        tm.sync();
        visible = o.op;
      }
      uint8_t* d = o.dst + o.op;
      team_copy(tm, d, lit + lp, ll);
      if (off >= ml) {
        for (uint64_t j = tm.lane(); j < ml; j += Team::size) {
          const uint64_t src = from + j;
          o.dst[o.op + ll + j] = src >= o.op ? lit[lp + (src - o.op)] : o.dst[src];
        }
      } else {
        // j mod off kept incrementally: j grows by the team size each round
        // (off < ml < 2^32, so this is 32-bit arithmetic and two divisions per
        // sequence instead of one 64-bit modulo per byte)
        const uint32_t off32 = off, step = Team::size % off32;
        uint32_t r = tm.lane() % off32;
        for (uint64_t j = tm.lane(); j < ml; j += Team::size) {
          const uint64_t src = from + r;
          o.dst[o.op + ll + j] = src >= o.op ? lit[lp + (src - o.op)] : o.dst[src];
          r += step;
          if (r >= off32) r -= off32;
        }
      }
      o.op += ll + ml;
      lp += ll;
    }
    if (br.bits() != 0) return kErrStream;
  }
  if (o.op + (lsize - lp) > o.cap) return kErrOutput;
  team_copy(tm, o.dst + o.op, lit + lp, lsize - lp);
  o.op += lsize - lp;
  tm.sync();
  return kOk;
}

// All frames in src[0, len) (zstd frames and skippable frames, back to back)
// into dst; *out_bytes receives the total decoded size.
template <class Team>
__host__ __device__ int32_t zstd_frames(const Team& tm, ZState& z, const uint8_t* src, uint64_t len, uint8_t* dst,
                                        uint64_t cap, uint8_t* lit_buf, uint64_t& out_bytes) {
  if (tm.lane() == 0) build_length_codes(z);
  tm.sync();
  Out o{dst, cap, 0, 0};
  uint64_t ip = 0;
  out_bytes = 0;
  if (len == 0) return kErrTruncated;
  while (ip < len) {
    if (len - ip < 4) return kErrTruncated;
    const uint32_t magic = (uint32_t)load_le(src + ip, 4, 0);
    if ((magic & 0xFFFFFFF0u) == 0x184D2A50u) {          // skippable frame
      if (len - ip < 8) return kErrTruncated;
      const uint64_t sz = (uint32_t)load_le(src + ip + 4, 4, 0);
      if (sz > len - ip - 8) return kErrTruncated;
      ip += 8 + sz;
      continue;
    }
    if (magic != 0xFD2FB528u) return kErrFormat;
    ip += 4;
    if (ip >= len) return kErrTruncated;
    const uint32_t fhd = src[ip++];
    const uint32_t fcs_flag = fhd >> 6, single = (fhd >> 5) & 1u, checksum = (fhd >> 2) & 1u, did = fhd & 3u;
    if (fhd & 8u) return kErrFormat;                     // reserved bit
    const uint32_t did_bytes = did == 3 ? 4u : did;
    const uint32_t fcs_bytes = fcs_flag == 0 ? single : fcs_flag == 1 ? 2u : fcs_flag == 2 ? 4u : 8u;
    const uint64_t hdr = (single ? 0u : 1u) + did_bytes + fcs_bytes;
    if (hdr > len - ip) return kErrTruncated;
    ip += single ? 0u : 1u;
    if (did_bytes && load_le(src + ip, did_bytes, 0) != 0) return kErrFormat;   // dictionaries: unsupported
    ip += did_bytes;
    uint64_t fcs = fcs_bytes ? load_le(src + ip, fcs_bytes, 0) : 0;
    if (fcs_bytes == 2) fcs += 256;
    ip += fcs_bytes;
    o.frame0 = o.op;
    if (tm.lane() == 0) z.huf_log = z.have_ll = z.have_ml = z.have_of = 0;
    tm.sync();
    Rep rep{1u, 4u, 8u};
    for (;;) {
      if (len - ip < 3) return kErrTruncated;
      const uint32_t bh = (uint32_t)load_le(src + ip, 3, 0);
      ip += 3;
      const uint32_t last = bh & 1u, type = (bh >> 1) & 3u, bsize = bh >> 3;
      if (type == 0) {                                   // raw block
        if (bsize > len - ip) return kErrTruncated;
        if (bsize > o.cap - o.op) return kErrOutput;
        team_copy(tm, o.dst + o.op, src + ip, bsize);
        o.op += bsize;
        ip += bsize;
      } else if (type == 1) {                            // RLE block
        if (ip >= len) return kErrTruncated;
        if (bsize > o.cap - o.op) return kErrOutput;
        team_fill(tm, o.dst + o.op, src[ip], bsize);
        o.op += bsize;
        ip += 1;
      } else if (type == 2) {
        if (bsize > len - ip) return kErrTruncated;
        if (bsize > kBlockMax) return kErrFormat;
        int32_t e;
        if (bsize <= kStageBytes) {     // bit reads then come from shared memory, not global memory
          team_copy(tm, z.stage, src + ip, bsize);
          tm.sync();
          e = zstd_block(tm, z, z.stage, bsize, o, rep, lit_buf);
        } else {
          e = zstd_block(tm, z, src + ip, bsize, o, rep, lit_buf);
        }
        if (e) return e;
        ip += bsize;
      } else {
        return kErrFormat;
      }
      tm.sync();
      if (last) break;
    }
    if (checksum) {
      if (len - ip < 4) return kErrTruncated;
      ip += 4;
    }
    if (fcs_bytes && o.op - o.frame0 != fcs) return kErrOutput;
  }
  out_bytes = o.op;
  return kOk;
}

}  // namespace bs_zstd
