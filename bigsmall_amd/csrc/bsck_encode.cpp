// Host encoder for BSCK, the decode engine's GPU-native chunked entropy-coded
// format. The byte layout is documented in bsck_decode.hip; this file produces it.
//
// Symbol model (per tensor):
//   bf16, plane_mode 1 (dense):   one symbol per exponent present; every
//                                 element also stores sign<<7|mantissa in the plane.
//   bf16, plane_mode 2 (compact): dense's exponent symbols plus up to
//                                 256-#exponents "exact word" symbols for words
//                                 frequent enough to beat 8 raw bits (zeros of a
//                                 sparse tensor, the few values of a norm vector).
//   bf16/bytes, plane_mode 0:     every distinct value is a symbol (<= 256).
//   bytes, plane_mode 3 (pairs):  fp8 e4m3 bytes taken two at a time: one symbol
//                                 per pair of 4-bit exponent fields (e0 | e1 << 4),
//                                 and one plane byte holding both sign and
//                                 mantissa fields (m0 | s1 << 3 | m1 << 4 | s0 << 7).
//                                 Needs an even element count.
// The encoder picks the smallest by estimated entropy unless a mode is forced.
//
// Two entropy coders share the layout (header byte 28, which also says where a
// tANS chunk keeps its initial states):
//   coder 0, rANS: 64*K interleaved 32-bit states per chunk (K = lanes / 64 per
//     wavefront lane; L = 2^16, M = 2^12, 16-bit renormalisation: the
//     reference's state machine, bigsmall/codecs/rans.py:115-162). State
//     v = g*64 + l (lane l, group g) codes element t*64K + l*K + g at step t.
//     States are walked from the last step back to the first, v descending
//     within a step, so the decoder consumes the renorm words step-ascending,
//     v-ascending.
//   coder 1, tANS: the same 64*K states, each a 12-bit table-ANS state X in
//     [0, 4096) (encoder state x = X + 4096). The table spreads symbol s's
//     f_s slots over the 4096 positions (slot i of the frequency-sorted order
//     at position i * 2563 mod 4096); position p holding the k-th occurrence
//     (in position order) of s decodes as {s, nb = 12 - floor(log2(f_s + k)),
//     newX = ((f_s + k) << nb) - 4096} and X' = newX + next nb bits. The
//     blob stores that 4096-entry table. Each element's bits (its nb state
//     bits, then in compact mode its 8 raw plane bits) are appended to one
//     LSB-first bit stream per chunk in chunk element order, which is the
//     decoder's order (steps ascending, then lanes, then the lane's states).
//     Coder 1 stores the chunk's initial states X as 64*K u32 words before
//     the stream (state v = g*64 + l); coder 2 stores them as 12-bit fields
//     at the head of the stream itself, in the same reading order (lane l's
//     state g at bit 12*(l*K + g)), which saves 2.5 bytes per state. A
//     coder-2 blob also extends to at least 256 bytes past its last chunk's
//     offset, so that every chunk has 256 readable bytes from its start.
//
// Chunk c holds elements of the tensor in 512-element units: a full chunk
// (c < nf = n / (lanes*steps)) holds units c, nf + c, 2nf + c, ..., so the
// chunks that a launch decodes side by side write neighbouring addresses; the
// last, partial chunk holds the tail [nf*lanes*steps, n) in order. The dense
// planes of the full chunks are interleaved the same way, per plane block, in
// one region before the chunks; the partial chunk keeps its plane inline. The
// plane region starts on a 256-byte boundary of the blob and blob lengths are
// multiples of 256, so blobs placed at 256-byte aligned addresses read whole
// cache lines. In pair mode an element is a pair of bytes throughout.
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <thread>
#include <vector>

#include "../../include/bigsmall_hip.h"

namespace {

constexpr uint8_t kVersion = 3;       // BSCK layout version
constexpr uint32_t kWave = 64;        // lanes of a wavefront
constexpr uint32_t kL = 1u << 16;
constexpr uint32_t kM = 4096;
// steps per dense-plane block: 8 for 64 or 128 states per chunk, 4 for 256
inline uint32_t block_steps(uint32_t lanes) { return lanes == 256 ? 4u : 8u; }
constexpr uint32_t kStepAlign = 16;   // steps per chunk: a multiple of two blocks
constexpr uint32_t kUnit = 512;       // elements per output interleave unit (divides lanes * kStepAlign)

// Tensor element holding element j of chunk c (nf full chunks of `per` elements).
inline uint64_t chunk_elem(uint64_t c, uint64_t j, uint64_t nf, uint64_t per) {
  return c < nf ? ((j / kUnit) * nf + c) * kUnit + j % kUnit : nf * per + j;
}

inline uint64_t pad16(uint64_t v) { return (v + 15) & ~uint64_t(15); }
inline uint64_t pad256(uint64_t v) { return (v + 255) & ~uint64_t(255); }

constexpr uint32_t kSpreadStep = 2563;   // 4096/2 + 4096/8 + 3, odd: slot i -> position i * 2563 mod 4096
constexpr uint32_t kTabSlots = 4096;      // tANS table positions (= kM)

struct Plan {
  int mode = 1;
  int coder = 0;                // 0 rANS, 1 tANS (u32 state array), 2 tANS (states at the stream head)
  uint32_t eb = 2;
  uint32_t nsym = 0;
  uint32_t value[256];
  uint32_t consume[256];
  uint32_t freq[256];
  uint32_t cum[256];
  std::vector<uint8_t> sym_of;  // element key (word, byte or pair-exponent byte) -> symbol
  // tANS: the decode table the blob stores, and where the encoder goes
  std::vector<uint32_t> dtab;     // position -> newX | nb << 12 | symbol << 16
  std::vector<uint16_t> enc_pos;  // enc_pos[cum[s] + k]: position of the k-th occurrence of s
  uint32_t top_bits[256];         // 12 - floor(log2 f_s)
};

// Pair mode (fp8 e4m3 bytes b0 = w & 0xFF, b1 = w >> 8 of a 16-bit element w):
// the symbol key is the two exponent fields, the plane byte the rest.
inline uint32_t pair_key(uint32_t w) { return ((w >> 3) & 0xFu) | ((w >> 7) & 0xF0u); }
inline uint8_t pair_plane(uint32_t w) {
  return (uint8_t)((w & 0x07u) | ((w >> 12) & 0x08u) | ((w >> 4) & 0x70u) | (w & 0x80u));
}
inline uint8_t bf16_plane(uint32_t w) { return (uint8_t)(((w >> 8) & 0x80u) | (w & 0x7Fu)); }

void put16(uint8_t* p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
void put32(uint8_t* p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i)); }
void put64(uint8_t* p, uint64_t v) { for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i)); }

// counts -> frequencies summing to kM, every present symbol >= 1: proportional
// rounding (half up), then +-1 corrections one at a time, each to the symbol
// where it costs the fewest bits. The cost of f -> f+1 is c*log2(1 + 1/f) saved,
// of f -> f-1 c*log2(1 + 1/(f-1)) lost; both are ranked by the integer
// proxies c/(2f+1) and c/(2f-1) (ln(1 + 1/f) ~ 1/(f + 1/2)), compared by
// cross-multiplication, ties to the lower index. Integer-only, so the GPU
// encoder (bsck_encode_gpu.hip) reproduces it exactly.
void quantise(const std::vector<uint64_t>& counts, uint32_t* freq) {
  const size_t k = counts.size();
  uint64_t total = 0;
  for (uint64_t c : counts) total += c;
  int64_t sum = 0;
  std::vector<int64_t> f(k);
  for (size_t i = 0; i < k; ++i) {
    int64_t v = (int64_t)((2 * counts[i] * kM + total) / (2 * total));
    if (v < 1) v = 1;
    f[i] = v;
    sum += v;
  }
  while (sum != (int64_t)kM) {
    const bool up = sum < (int64_t)kM;
    size_t best = k;
    for (size_t i = 0; i < k; ++i) {
      if (!up && f[i] <= 1) continue;
      if (best == k) { best = i; continue; }
      const uint64_t di = up ? 2 * f[i] + 1 : 2 * f[i] - 1, db = up ? 2 * f[best] + 1 : 2 * f[best] - 1;
      // counts < 2^50 and d <= 8193: the products fit in 64 bits
      const uint64_t lhs = counts[i] * db, rhs = counts[best] * di;
      if (up ? lhs > rhs : lhs < rhs) best = i;     // up: largest c/(2f+1); down: smallest c/(2f-1)
    }
    if (up) { f[best]++; sum++; }
    else { f[best]--; sum--; }
  }
  for (size_t i = 0; i < k; ++i) freq[i] = (uint32_t)f[i];
}

double entropy_bits(const std::vector<uint64_t>& counts) {
  uint64_t total = 0;
  for (uint64_t c : counts) total += c;
  double h = 0;
  for (uint64_t c : counts) if (c) h += (double)c * std::log2((double)total / (double)c);
  return h;
}

template <typename Fn>
void parallel_for(uint64_t n, int threads, Fn fn) {
  if (threads <= 1 || n <= 1) { for (uint64_t i = 0; i < n; ++i) fn(i); return; }
  std::atomic<uint64_t> next{0};
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t)
    pool.emplace_back([&] { for (uint64_t i; (i = next.fetch_add(1)) < n;) fn(i); });
  for (auto& th : pool) th.join();
}

std::vector<uint64_t> histogram(const void* src, uint64_t n, uint32_t eb, int threads) {
  const uint32_t bins = eb == 2 ? 65536u : 256u;
  const uint64_t parts = std::max<uint64_t>(1, std::min<uint64_t>((uint64_t)threads, n / (1u << 20) + 1));
  std::vector<std::vector<uint64_t>> part(parts, std::vector<uint64_t>(bins, 0));
  parallel_for(parts, threads, [&](uint64_t p) {
    uint64_t lo = n * p / parts, hi = n * (p + 1) / parts;
    auto& h = part[p];
    if (eb == 2) { const uint16_t* w = (const uint16_t*)src; for (uint64_t i = lo; i < hi; ++i) h[w[i]]++; }
    else { const uint8_t* w = (const uint8_t*)src; for (uint64_t i = lo; i < hi; ++i) h[w[i]]++; }
  });
  std::vector<uint64_t> h(bins, 0);
  for (auto& q : part) for (uint32_t i = 0; i < bins; ++i) h[i] += q[i];
  return h;
}

// tANS tables from the quantised frequencies: symbol s owns slots
// [cum_s, cum_s + f_s) of the sorted order, slot i sits at position
// i * kSpreadStep mod 4096, and the positions of s numbered in increasing
// order give its k-th occurrence.
void build_tans(Plan& P) {
  std::vector<uint8_t> at(kTabSlots);
  for (uint32_t s = 0; s < P.nsym; ++s)
    for (uint32_t k = 0; k < P.freq[s]; ++k) at[((P.cum[s] + k) * kSpreadStep) & (kTabSlots - 1)] = (uint8_t)s;
  P.dtab.assign(kTabSlots, 0);
  P.enc_pos.assign(kTabSlots, 0);
  uint32_t seen[256] = {0};
  for (uint32_t p = 0; p < kTabSlots; ++p) {
    const uint32_t s = at[p], k = seen[s]++, next = P.freq[s] + k;   // next in [f, 2f)
    uint32_t nb = 0;
    while ((next << nb) < kTabSlots) ++nb;                             // 12 - floor(log2 next)
    P.dtab[p] = ((next << nb) - kTabSlots) | (nb << 12) | (s << 16);
    P.enc_pos[P.cum[s] + k] = (uint16_t)p;
  }
  for (uint32_t s = 0; s < P.nsym; ++s) {
    uint32_t b = 0;
    while ((P.freq[s] << b) < kTabSlots) ++b;
    P.top_bits[s] = b;                                                 // 12 - floor(log2 f)
  }
}

// `hist`: element histogram (65536 words for bf16, 256 bytes for fp8);
// `pair_hist`: for fp8 with an even count, the histogram of byte pairs as
// 16-bit words (null otherwise).
bool make_plan(const std::vector<uint64_t>& hist, const std::vector<uint64_t>* pair_hist, uint32_t eb, int forced,
               int coder, Plan& P) {
  P.eb = eb;
  P.coder = coder;
  std::vector<uint64_t> cnt;
  if (eb == 1) {
    if (forced != BS_CHUNK_MODE_AUTO && forced != 0 && forced != 3) return false;
    if (forced == 3 && !pair_hist) return false;
    std::vector<uint64_t> bc;
    for (uint32_t v = 0; v < 256; ++v) if (hist[v]) bc.push_back(hist[v]);
    const double cost_bytes = entropy_bits(bc);
    uint64_t pc[256] = {0}, pairs = 0;
    double cost_pairs = 1e300;
    if (pair_hist) {
      for (uint32_t w = 0; w < 65536; ++w) if ((*pair_hist)[w]) { pc[pair_key(w)] += (*pair_hist)[w]; pairs += (*pair_hist)[w]; }
      std::vector<uint64_t> c;
      for (uint32_t k = 0; k < 256; ++k) if (pc[k]) c.push_back(pc[k]);
      cost_pairs = entropy_bits(c) + 8.0 * (double)pairs;
    }
    // pairs decode one symbol per two elements (about the dense bf16 rate per
    // symbol), so they are taken unless their entropy estimate is 2 % above
    // that of byte symbols (for fp8 e4m3 of N(0, 1) it is 1.1 % above, and
    // the blobs differ by -0.5 to +0.6 %: pairs also halve the chunks' states)
    P.mode = forced != BS_CHUNK_MODE_AUTO ? forced : (cost_pairs <= cost_bytes * 1.02 ? 3 : 0);
    if (P.mode == 0) {
      P.sym_of.assign(256, 0);
      for (uint32_t v = 0; v < 256; ++v) if (hist[v]) {
        P.sym_of[v] = (uint8_t)P.nsym; P.value[P.nsym] = v; P.consume[P.nsym] = 0;
        cnt.push_back(hist[v]); P.nsym++;
      }
    } else {
      P.sym_of.assign(256, 0);
      for (uint32_t k = 0; k < 256; ++k) if (pc[k]) {
        P.sym_of[k] = (uint8_t)P.nsym; P.value[P.nsym] = k; P.consume[P.nsym] = 1;
        cnt.push_back(pc[k]); P.nsym++;
      }
    }
    quantise(cnt, P.freq);
  } else {
    P.sym_of.assign(hist.size(), 0);
    uint64_t ecnt[256] = {0};
    uint32_t unique = 0;
    for (uint32_t w = 0; w < 65536; ++w) if (hist[w]) { ecnt[(w >> 7) & 0xFF] += hist[w]; unique++; }
    uint32_t nexp = 0;
    for (int e = 0; e < 256; ++e) nexp += ecnt[e] != 0;
    uint64_t N = 0; for (uint64_t c : hist) N += c;

    // dense
    std::vector<uint64_t> dense_c;
    for (int e = 0; e < 256; ++e) if (ecnt[e]) dense_c.push_back(ecnt[e]);
    const double cost_dense = entropy_bits(dense_c) + 8.0 * (double)N;
    // exact-value (mode 0)
    double cost_exact = 1e300;
    if (unique <= 256) {
      std::vector<uint64_t> c; for (uint32_t w = 0; w < 65536; ++w) if (hist[w]) c.push_back(hist[w]);
      cost_exact = entropy_bits(c);
    }
    // compact: exact words worth more than ~1 bit per occurrence
    std::vector<std::pair<double, uint32_t>> cand;
    for (uint32_t w = 0; w < 65536; ++w) {
      if (hist[w] < 2) continue;
      double save = 8.0 + std::log2((double)hist[w] / (double)ecnt[(w >> 7) & 0xFF]);
      if (save > 1.0) cand.push_back({save * (double)hist[w], w});
    }
    std::sort(cand.begin(), cand.end(), [](auto& a, auto& b) { return a.first > b.first || (a.first == b.first && a.second < b.second); });
    std::vector<uint8_t> is_exact(65536, 0);
    uint32_t room = 256 - nexp, taken = 0;
    for (auto& c : cand) { if (taken == room) break; is_exact[c.second] = 1; taken++; }
    uint64_t rest[256] = {0};
    std::vector<uint64_t> comp_c;
    for (uint32_t w = 0; w < 65536; ++w) if (hist[w]) { if (is_exact[w]) comp_c.push_back(hist[w]); else rest[(w >> 7) & 0xFF] += hist[w]; }
    uint64_t plane_n = 0;
    for (int e = 0; e < 256; ++e) if (rest[e]) { comp_c.push_back(rest[e]); plane_n += rest[e]; }
    const double cost_comp = taken ? entropy_bits(comp_c) + 8.0 * (double)plane_n : 1e300;

    int mode = forced;
    if (mode == BS_CHUNK_MODE_AUTO) {
      if (cost_exact <= cost_dense && cost_exact <= cost_comp) mode = 0;
      else if (cost_comp < cost_dense * 0.995) mode = 2;
      else mode = 1;
    }
    if (mode == 0 && unique > 256) return false;
    if (mode < 0 || mode > 2) return false;
    P.mode = mode;
    if (mode == 0) {
      for (uint32_t w = 0; w < 65536; ++w) if (hist[w]) {
        P.sym_of[w] = (uint8_t)P.nsym; P.value[P.nsym] = w; P.consume[P.nsym] = 0;
        cnt.push_back(hist[w]); P.nsym++;
      }
    } else {
      if (mode == 1) std::fill(is_exact.begin(), is_exact.end(), 0);
      int sym_of_exp[256];
      for (int e = 0; e < 256; ++e) sym_of_exp[e] = -1;
      uint64_t cls[256] = {0};
      for (uint32_t w = 0; w < 65536; ++w) if (hist[w] && !is_exact[w]) cls[(w >> 7) & 0xFF] += hist[w];
      for (int e = 0; e < 256; ++e) if (cls[e]) {
        sym_of_exp[e] = (int)P.nsym; P.value[P.nsym] = (uint32_t)e << 7; P.consume[P.nsym] = 1;
        cnt.push_back(cls[e]); P.nsym++;
      }
      for (uint32_t w = 0; w < 65536; ++w) {
        if (!hist[w]) continue;
        if (is_exact[w]) {
          P.sym_of[w] = (uint8_t)P.nsym; P.value[P.nsym] = w; P.consume[P.nsym] = 0;
          cnt.push_back(hist[w]); P.nsym++;
        } else P.sym_of[w] = (uint8_t)sym_of_exp[(w >> 7) & 0xFF];
      }
    }
    quantise(cnt, P.freq);
  }
  uint32_t c = 0;
  for (uint32_t s = 0; s < P.nsym; ++s) { P.cum[s] = c; c += P.freq[s]; }
  if (c != kM || P.nsym < 1 || P.nsym > 256) return false;
  if (coder != 0) build_tans(P);
  return true;
}

// Symbols and plane bytes of a chunk's elements (src holds the chunk's nc
// elements in chunk order: 16-bit words for bf16 and pair mode, bytes else).
void chunk_symbols(const Plan& P, const void* src, uint32_t nc, std::vector<uint8_t>& sym,
                   std::vector<uint8_t>& plane) {
  sym.resize(nc);
  plane.assign(nc, 0);
  const uint16_t* w16 = (const uint16_t*)src;
  const uint8_t* w8 = (const uint8_t*)src;
  for (uint32_t j = 0; j < nc; ++j) {
    if (P.mode == 3) {
      sym[j] = P.sym_of[pair_key(w16[j])];
      plane[j] = pair_plane(w16[j]);
    } else if (P.eb == 2) {
      sym[j] = P.sym_of[w16[j]];
      plane[j] = bf16_plane(w16[j]);
    } else {
      sym[j] = P.sym_of[w8[j]];
    }
  }
}

// The dense plane (modes 1 and 3): per block of bs steps, wavefront lane l's
// bs*K bytes are contiguous, step-major: byte (q, g) of lane l at l*bs*K + q*K + g.
std::vector<uint8_t> dense_plane(const std::vector<uint8_t>& plane, uint32_t nc, uint32_t lanes) {
  const uint32_t nsteps = (nc + lanes - 1) / lanes, K = lanes / kWave, bs = block_steps(lanes);
  const uint32_t nblk = (nsteps + bs - 1) / bs;
  std::vector<uint8_t> out((size_t)nblk * bs * lanes, 0);
  for (uint32_t j = 0; j < nc; ++j) {
    const uint32_t t = j / lanes, r = j % lanes, l = r / K, g = r % K;
    out[(size_t)(t / bs) * bs * lanes + l * bs * K + (t % bs) * K + g] = plane[j];
  }
  return out;
}

// rANS: states | words (16-padded) | plane (16-padded, or to *plane_out).
// `lanes` = 64*K interleaved states; state v = g*64 + l is group g of
// wavefront lane l. Step t covers chunk elements t*lanes .. t*lanes+lanes-1.
void encode_chunk_rans(const Plan& P, const std::vector<uint8_t>& sym, const std::vector<uint8_t>& pb, uint32_t nc,
                       uint32_t lanes, uint32_t& n_words, uint32_t& n_plane, std::vector<uint8_t>& out,
                       std::vector<uint8_t>* plane_out) {
  const uint32_t nsteps = (nc + lanes - 1) / lanes;
  const uint32_t K = lanes / kWave;
  std::vector<uint16_t> words(nc + 1);
  size_t pos = words.size();
  std::vector<uint32_t> x(lanes, kL);
  uint64_t xmax[256];
  for (uint32_t s = 0; s < P.nsym; ++s) xmax[s] = (uint64_t)P.freq[s] << 20;
  auto elem = [&](uint32_t t, uint32_t v) -> uint64_t { return (uint64_t)t * lanes + (v % kWave) * K + v / kWave; };
  for (uint32_t t = nsteps; t-- > 0;) {
    for (uint32_t v = lanes; v-- > 0;) {
      const uint64_t j = elem(t, v);
      if (j >= nc) continue;
      const uint32_t s = sym[j], f = P.freq[s];
      uint32_t xv = x[v];
      if ((uint64_t)xv >= xmax[s]) { words[--pos] = (uint16_t)(xv & 0xFFFF); xv >>= 16; }
      const uint32_t q = xv / f;
      x[v] = (q << 12) + (xv - q * f) + P.cum[s];
    }
  }
  n_words = (uint32_t)(words.size() - pos);
  std::vector<uint8_t> plane;
  if (P.mode == 1 || P.mode == 3) {
    plane = dense_plane(pb, nc, lanes);
  } else if (P.mode == 2) {
    // compact plane: bytes of consuming elements in decode order (step, then v)
    plane.reserve(nc);
    for (uint32_t t = 0; t < nsteps; ++t)
      for (uint32_t v = 0; v < lanes; ++v) {
        const uint64_t j = elem(t, v);
        if (j < nc && P.consume[sym[j]]) plane.push_back(pb[j]);
      }
  }
  n_plane = (uint32_t)plane.size();
  const uint64_t wb = pad16((uint64_t)n_words * 2), pbytes = plane_out ? 0 : pad16(n_plane);
  out.assign(4 * lanes + wb + pbytes, 0);
  for (uint32_t l = 0; l < lanes; ++l) put32(out.data() + 4 * l, x[l]);
  for (uint32_t i = 0; i < n_words; ++i) put16(out.data() + 4 * lanes + 2 * i, words[pos + i]);
  if (plane_out) plane_out->swap(plane);
  else if (n_plane) memcpy(out.data() + 4 * lanes + wb, plane.data(), n_plane);
}

// tANS: [coder 1: states, u32 X each] | bit stream (whole u32 words,
// 16-padded; coder 2: the states' 12-bit fields first) | plane (modes 1 and
// 3; 16-padded, or to *plane_out). n_bits = the stream's length in bits;
// compact mode keeps its plane bytes in the stream.
void encode_chunk_tans(const Plan& P, const std::vector<uint8_t>& sym, const std::vector<uint8_t>& pb, uint32_t nc,
                       uint32_t lanes, uint32_t& n_bits, uint32_t& n_plane, std::vector<uint8_t>& out,
                       std::vector<uint8_t>* plane_out) {
  const bool head = P.coder == 2;
  const uint32_t nsteps = (nc + lanes - 1) / lanes;
  std::vector<uint32_t> field(nc);       // element j's bits, LSB first
  std::vector<uint8_t> width(nc);
  std::vector<uint32_t> x(lanes, kTabSlots);  // encoder states in [4096, 8192)
  const uint32_t K = lanes / kWave;
  for (uint32_t t = nsteps; t-- > 0;) {
    for (uint32_t v = lanes; v-- > 0;) {
      const uint64_t j = (uint64_t)t * lanes + (v % kWave) * K + v / kWave;
      if (j >= nc) continue;
      const uint32_t s = sym[j], f = P.freq[s], tb = P.top_bits[s];
      const uint32_t nb = tb - (x[v] < (f << tb) ? 1u : 0u);      // (x >> nb) in [f, 2f)
      uint32_t bits = x[v] & ((1u << nb) - 1u), w = nb;
      x[v] = kTabSlots + P.enc_pos[P.cum[s] + (x[v] >> nb) - f];
      if (P.mode == 2 && P.consume[s]) { bits |= (uint32_t)pb[j] << nb; w += 8; }
      field[j] = bits;
      width[j] = (uint8_t)w;
    }
  }
  uint64_t total = head ? 12ull * lanes : 0;
  for (uint32_t j = 0; j < nc; ++j) total += width[j];
  n_bits = (uint32_t)total;
  const uint64_t sbytes = pad16(((total + 31) / 32) * 4);
  std::vector<uint8_t> plane;
  if (P.mode == 1 || P.mode == 3) plane = dense_plane(pb, nc, lanes);
  n_plane = (uint32_t)plane.size();
  const uint64_t pbytes = plane_out ? 0 : pad16(n_plane);
  const uint32_t sarr = head ? 0u : 4 * lanes;   // bytes of the u32 state array
  out.assign(sarr + sbytes + pbytes, 0);
  if (!head)
    for (uint32_t l = 0; l < lanes; ++l) put32(out.data() + 4 * l, x[l] - kTabSlots);
  uint8_t* bs = out.data() + sarr;
  uint64_t acc = 0;                       // pending bits, LSB first
  uint32_t pending = 0;
  if (head) {
    for (uint32_t i = 0; i < lanes; ++i) {  // reading order i = l*K + g: state v = g*64 + l
      acc |= (uint64_t)(x[(i % K) * kWave + i / K] - kTabSlots) << pending;
      pending += 12;
      if (pending >= 32) { put32(bs, (uint32_t)acc); bs += 4; acc >>= 32; pending -= 32; }
    }
  }
  for (uint32_t j = 0; j < nc; ++j) {     // chunk element order is the decoder's reading order
    acc |= (uint64_t)field[j] << pending; // < 2^52: pending < 32, fields of at most 20 bits
    pending += width[j];
    if (pending >= 32) { put32(bs, (uint32_t)acc); bs += 4; acc >>= 32; pending -= 32; }
  }
  if (pending) put32(bs, (uint32_t)acc);
  if (plane_out) plane_out->swap(plane);
  else if (n_plane) memcpy(out.data() + sarr + sbytes, plane.data(), n_plane);
}

}  // namespace

extern "C" {

static bool lanes_ok(uint32_t lanes) { return lanes == 64 || lanes == 128 || lanes == 256; }
// A chunk holds at most 2^24 elements (the decoder refuses larger), so every
// byte offset inside a chunk fits 32 bits.
static bool chunk_ok(uint32_t lanes, uint32_t steps) { return (uint64_t)lanes * steps <= (1ull << 24); }

int bs_chunk_encode_bound_ex(uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, int32_t coder,
                             uint64_t* bound) {
  if (!bound || (elem_bytes != 1 && elem_bytes != 2) || steps == 0 || steps % kStepAlign || !lanes_ok(lanes) ||
      !chunk_ok(lanes, steps) || coder < 0 || coder > 2)
    return BS_ERR_ARG;
  const uint64_t per = (uint64_t)lanes * steps;
  const uint64_t nch = (n + per - 1) / per;
  // per element at most one 16-bit word (rANS) or 20 bits (tANS), and one
  // plane byte; per state 4 bytes (rANS, tANS coder 1) or 12 bits (coder 2);
  // and the coder-2 tail of up to 256 bytes after the last chunk
  const uint64_t stream = coder == 0 ? pad16(2 * per) : pad16(((per * 20 + 12ull * lanes + 31) / 32) * 4);
  *bound = pad16(32 + 4 * 256) + (coder != 0 ? 4 * kTabSlots : 0) + 16 * nch +
           nch * (4 * lanes + stream + pad16(per) + 32) + 512 + 256;
  return BS_OK;
}

int bs_chunk_encode_bound(uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, uint64_t* bound) {
  return bs_chunk_encode_bound_ex(n, elem_bytes, lanes, steps, 0, bound);
}

int bs_chunk_encode_ex(const void* src, uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, int32_t mode,
                       int32_t coder, uint8_t* dst, uint64_t cap, uint64_t* out_len, int n_threads) {
  if (!out_len || (elem_bytes != 1 && elem_bytes != 2) || steps == 0 || steps % kStepAlign || !lanes_ok(lanes) ||
      !chunk_ok(lanes, steps) || coder < 0 || coder > 2)
    return BS_ERR_ARG;
  if (n == 0) { *out_len = 0; return BS_OK; }
  if (!src || !dst) return BS_ERR_ARG;
  if (n_threads < 1) n_threads = 1;
  std::vector<uint64_t> hist = histogram(src, n, elem_bytes, n_threads);
  std::vector<uint64_t> pair_hist;
  const bool pairs_ok = elem_bytes == 1 && n % 2 == 0 && (mode == BS_CHUNK_MODE_AUTO || mode == 3);
  if (pairs_ok) pair_hist = histogram(src, n / 2, 2, n_threads);
  Plan P;
  if (!make_plan(hist, pairs_ok ? &pair_hist : nullptr, elem_bytes, mode, coder, P)) return BS_ERR_ARG;

  // pair mode codes 16-bit elements (byte pairs): the chunk geometry counts them
  const uint32_t ew = P.mode == 3 ? 2u : elem_bytes;        // bytes per coded element
  const uint64_t ne = n * elem_bytes / ew;
  const uint64_t per = (uint64_t)lanes * steps;
  const uint64_t nch64 = (ne + per - 1) / per;
  if (nch64 > 0xFFFFFFFFull) return BS_ERR_ARG;
  const uint32_t nch = (uint32_t)nch64;
  const uint64_t nf = ne / per;                       // full chunks
  const bool split_plane = P.mode == 1 || P.mode == 3;   // full chunks' dense planes go to the plane region
  const uint64_t stab = pad16(32 + 4ull * P.nsym);
  const uint64_t ctab = stab + (coder != 0 ? 4ull * kTabSlots : 0);   // tANS: the decode table first
  const uint64_t preg = pad256(ctab + 16ull * nch);  // plane region: nf*per bytes in modes 1 and 3
  const uint64_t pblk = (uint64_t)block_steps(lanes) * lanes;   // plane bytes per block
  std::vector<std::vector<uint8_t>> chunks(nch);
  std::vector<uint32_t> nw(nch), np(nch);
  std::vector<uint8_t> plane_region(split_plane ? nf * per : 0);
  parallel_for(nch, n_threads, [&](uint64_t c) {
    const uint32_t nc = (uint32_t)std::min<uint64_t>(per, ne - c * per);
    std::vector<uint8_t> gathered((size_t)nc * ew);   // the chunk's elements in chunk order
    for (uint32_t j = 0; j < nc; j += (c < nf ? kUnit : nc))
      memcpy(gathered.data() + (size_t)j * ew, (const uint8_t*)src + chunk_elem(c, j, nf, per) * ew,
             (size_t)std::min<uint32_t>(c < nf ? kUnit : nc, nc - j) * ew);
    std::vector<uint8_t> sym, pb, plane;
    chunk_symbols(P, gathered.data(), nc, sym, pb);
    const bool split = split_plane && c < nf;
    if (coder == 0) encode_chunk_rans(P, sym, pb, nc, lanes, nw[c], np[c], chunks[c], split ? &plane : nullptr);
    else encode_chunk_tans(P, sym, pb, nc, lanes, nw[c], np[c], chunks[c], split ? &plane : nullptr);
    if (split)
      for (uint64_t b = 0; b * pblk < plane.size(); ++b)
        memcpy(plane_region.data() + (b * nf + c) * pblk, plane.data() + b * pblk, pblk);
  });

  uint64_t total = preg + plane_region.size();
  std::vector<uint64_t> offs(nch);
  for (uint32_t c = 0; c < nch; ++c) { offs[c] = total; total += chunks[c].size(); }
  const uint64_t end = total;
  // blob lengths are multiples of 256; coder 2: 256 bytes at least from the last chunk's start
  total = pad256(coder == 2 ? std::max(total, offs[nch - 1] + 256) : total);
  if (total > cap) return BS_ERR_CAP;
  memset(dst, 0, preg);
  memcpy(dst, "BSCK", 4);
  dst[4] = kVersion; dst[5] = (uint8_t)elem_bytes; dst[6] = (uint8_t)P.mode; dst[7] = 12;
  put64(dst + 8, n); put32(dst + 16, steps); put16(dst + 20, lanes); put16(dst + 22, P.nsym);
  put32(dst + 24, nch); put32(dst + 28, (uint32_t)coder);
  for (uint32_t s = 0; s < P.nsym; ++s)
    put32(dst + 32 + 4 * s, (P.value[s] & 0xFFFF) | (P.freq[s] << 16) | (P.consume[s] << 31));
  if (coder != 0)
    for (uint32_t p = 0; p < kTabSlots; ++p) put32(dst + stab + 4 * p, P.dtab[p]);
  for (uint32_t c = 0; c < nch; ++c) {
    put64(dst + ctab + 16ull * c, offs[c]);
    put32(dst + ctab + 16ull * c + 8, nw[c]);
    put32(dst + ctab + 16ull * c + 12, np[c]);
  }
  memset(dst + end, 0, total - end);
  if (!plane_region.empty()) memcpy(dst + preg, plane_region.data(), plane_region.size());
  parallel_for(nch, n_threads, [&](uint64_t c) { memcpy(dst + offs[c], chunks[c].data(), chunks[c].size()); });
  *out_len = total;
  return BS_OK;
}

int bs_chunk_encode(const void* src, uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, int32_t mode,
                    uint8_t* dst, uint64_t cap, uint64_t* out_len, int n_threads) {
  return bs_chunk_encode_ex(src, n, elem_bytes, lanes, steps, mode, 0, dst, cap, out_len, n_threads);
}

}  // extern "C"
