// Host encoder for BSCK, the decode engine's GPU-native chunked rANS format.
// The byte layout is documented in bsck_decode.hip; this file produces it.
//
// Symbol model (per tensor):
//   bf16, plane_mode 1 (dense):   one symbol per exponent present; every
//                                 element also stores sign<<7|mantissa in the plane.
//   bf16, plane_mode 2 (compact): dense's exponent symbols plus up to
//                                 256-#exponents "exact word" symbols for words
//                                 frequent enough to beat 8 raw bits (zeros of a
//                                 sparse tensor, the few values of a norm vector).
//   bf16/bytes, plane_mode 0:     every distinct value is a symbol (<= 256).
// The encoder picks the smallest by estimated entropy unless a mode is forced.
//
// rANS encoding per chunk: 64*K interleaved 32-bit states (K = 1 or 2 per
// wavefront lane; L = 2^16, M = 2^12, 16-bit renormalisation: the reference's
// state machine, bigsmall/codecs/rans.py:115-162). State v = g*64 + l (lane l,
// group g) codes element t*64K + l*K + g at step t. States are walked from the
// last step back to the first, v descending within a step, so the decoder
// consumes the renorm words step-ascending, v-ascending.
//
// Chunk c holds elements of the tensor in 512-element units: a full chunk
// (c < nf = n / (lanes*steps)) holds units c, nf + c, 2nf + c, ..., so the
// chunks that a launch decodes side by side write neighbouring addresses; the
// last, partial chunk holds the tail [nf*lanes*steps, n) in order. The dense
// planes of the full chunks are interleaved the same way, per plane block, in
// one region before the chunks; the partial chunk keeps its plane inline. The
// plane region starts on a 256-byte boundary of the blob and blob lengths are
// multiples of 256, so blobs placed at 256-byte aligned addresses read whole
// cache lines.
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

struct Plan {
  int mode = 1;
  uint32_t eb = 2;
  uint32_t nsym = 0;
  uint32_t value[256];
  uint32_t consume[256];
  uint32_t freq[256];
  uint32_t cum[256];
  std::vector<uint8_t> sym_of;  // word (or byte) -> symbol
};

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

bool make_plan(const std::vector<uint64_t>& hist, uint32_t eb, int forced, Plan& P) {
  P.eb = eb;
  P.sym_of.assign(hist.size(), 0);
  std::vector<uint64_t> cnt;
  if (eb == 1) {
    if (forced != BS_CHUNK_MODE_AUTO && forced != 0) return false;
    P.mode = 0;
    for (uint32_t v = 0; v < 256; ++v) if (hist[v]) {
      P.sym_of[v] = (uint8_t)P.nsym; P.value[P.nsym] = v; P.consume[P.nsym] = 0;
      cnt.push_back(hist[v]); P.nsym++;
    }
    quantise(cnt, P.freq);
  } else {
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
  return c == kM && P.nsym >= 1 && P.nsym <= 256;
}

// Encode one chunk, whose nc elements are src[0..nc), into `out` (states |
// words | plane, each 16-padded; the plane goes to *plane_out instead when
// that is given). `lanes` = 64*K interleaved states; virtual lane v = g*64 + l
// is state group g of wavefront lane l. Step t covers chunk elements
// t*lanes .. t*lanes+lanes-1.
void encode_chunk(const Plan& P, const void* src, uint32_t nc, uint32_t lanes, uint32_t& n_words, uint32_t& n_plane,
                  std::vector<uint8_t>& out, std::vector<uint8_t>* plane_out) {
  const uint32_t nsteps = (nc + lanes - 1) / lanes;
  const uint32_t K = lanes / kWave;
  std::vector<uint16_t> words(nc + 1);
  size_t pos = words.size();
  std::vector<uint32_t> x(lanes, kL);
  const uint16_t* w16 = (const uint16_t*)src;
  const uint8_t* w8 = (const uint8_t*)src;
  auto sym_at = [&](uint64_t j) -> uint32_t { return P.sym_of[P.eb == 2 ? w16[j] : w8[j]]; };
  uint64_t xmax[256];
  for (uint32_t s = 0; s < P.nsym; ++s) xmax[s] = (uint64_t)P.freq[s] << 20;
  auto elem = [&](uint32_t t, uint32_t v) -> uint64_t { return (uint64_t)t * lanes + (v % kWave) * K + v / kWave; };
  for (uint32_t t = nsteps; t-- > 0;) {
    for (uint32_t v = lanes; v-- > 0;) {
      const uint64_t j = elem(t, v);
      if (j >= nc) continue;
      const uint32_t s = sym_at(j), f = P.freq[s];
      uint32_t xv = x[v];
      if ((uint64_t)xv >= xmax[s]) { words[--pos] = (uint16_t)(xv & 0xFFFF); xv >>= 16; }
      const uint32_t q = xv / f;
      x[v] = (q << 12) + (xv - q * f) + P.cum[s];
    }
  }
  n_words = (uint32_t)(words.size() - pos);
  std::vector<uint8_t> plane;
  if (P.mode == 1) {
    // dense plane: per 8-step block, wavefront lane l's 8*K bytes are contiguous,
    // step-major: byte (q, g) of lane l at l*8K + q*K + g
    const uint32_t bs = block_steps(lanes);
    const uint32_t nblk = (nsteps + bs - 1) / bs;
    plane.assign((size_t)nblk * bs * lanes, 0);
    for (uint32_t j = 0; j < nc; ++j) {
      const uint32_t w = w16[j], t = j / lanes, r = j % lanes, l = r / K, g = r % K;
      plane[(size_t)(t / bs) * bs * lanes + l * bs * K + (t % bs) * K + g] =
          (uint8_t)(((w >> 8) & 0x80) | (w & 0x7F));
    }
  } else if (P.mode == 2) {
    // compact plane: bytes of consuming elements in decode order (step, then v)
    plane.reserve(nc);
    for (uint32_t t = 0; t < nsteps; ++t)
      for (uint32_t v = 0; v < lanes; ++v) {
        const uint64_t j = elem(t, v);
        if (j >= nc) continue;
        const uint32_t w = w16[j];
        if (P.consume[P.sym_of[w]]) plane.push_back((uint8_t)(((w >> 8) & 0x80) | (w & 0x7F)));
      }
  }
  n_plane = (uint32_t)plane.size();
  const uint64_t wb = pad16((uint64_t)n_words * 2), pb = plane_out ? 0 : pad16(n_plane);
  out.assign(4 * lanes + wb + pb, 0);
  for (uint32_t l = 0; l < lanes; ++l) put32(out.data() + 4 * l, x[l]);
  for (uint32_t i = 0; i < n_words; ++i) put16(out.data() + 4 * lanes + 2 * i, words[pos + i]);
  if (plane_out) plane_out->swap(plane);
  else if (n_plane) memcpy(out.data() + 4 * lanes + wb, plane.data(), n_plane);
}

}  // namespace

extern "C" {

static bool lanes_ok(uint32_t lanes) { return lanes == 64 || lanes == 128 || lanes == 256; }
// A chunk holds at most 2^24 elements (the decoder refuses larger), so every
// byte offset inside a chunk fits 32 bits.
static bool chunk_ok(uint32_t lanes, uint32_t steps) { return (uint64_t)lanes * steps <= (1ull << 24); }

int bs_chunk_encode_bound(uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, uint64_t* bound) {
  if (!bound || (elem_bytes != 1 && elem_bytes != 2) || steps == 0 || steps % kStepAlign || !lanes_ok(lanes) ||
      !chunk_ok(lanes, steps))
    return BS_ERR_ARG;
  const uint64_t per = (uint64_t)lanes * steps;
  const uint64_t nch = (n + per - 1) / per;
  *bound = pad16(32 + 4 * 256) + 16 * nch + nch * (4 * lanes + pad16(2 * per) + pad16(per) + 32) + 512;
  return BS_OK;
}

int bs_chunk_encode(const void* src, uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, int32_t mode,
                    uint8_t* dst, uint64_t cap, uint64_t* out_len, int n_threads) {
  if (!out_len || (elem_bytes != 1 && elem_bytes != 2) || steps == 0 || steps % kStepAlign || !lanes_ok(lanes) ||
      !chunk_ok(lanes, steps))
    return BS_ERR_ARG;
  if (n == 0) { *out_len = 0; return BS_OK; }
  if (!src || !dst) return BS_ERR_ARG;
  if (n_threads < 1) n_threads = 1;
  std::vector<uint64_t> hist = histogram(src, n, elem_bytes, n_threads);
  Plan P;
  if (!make_plan(hist, elem_bytes, mode, P)) return BS_ERR_ARG;

  const uint64_t per = (uint64_t)lanes * steps;
  const uint64_t nch64 = (n + per - 1) / per;
  if (nch64 > 0xFFFFFFFFull) return BS_ERR_ARG;
  const uint32_t nch = (uint32_t)nch64;
  const uint64_t nf = n / per;                       // full chunks
  const bool split_plane = P.mode == 1;              // full chunks' dense planes go to the plane region
  const uint64_t ctab = pad16(32 + 4ull * P.nsym);
  const uint64_t preg = pad256(ctab + 16ull * nch);  // plane region: nf*per bytes in mode 1
  const uint64_t pblk = (uint64_t)block_steps(lanes) * lanes;   // plane bytes per block
  std::vector<std::vector<uint8_t>> chunks(nch);
  std::vector<uint32_t> nw(nch), np(nch);
  std::vector<uint8_t> plane_region(split_plane ? nf * per : 0);
  parallel_for(nch, n_threads, [&](uint64_t c) {
    const uint32_t nc = (uint32_t)std::min<uint64_t>(per, n - c * per);
    std::vector<uint8_t> gathered((size_t)nc * elem_bytes);   // the chunk's elements in chunk order
    for (uint32_t j = 0; j < nc; j += (c < nf ? kUnit : nc))
      memcpy(gathered.data() + (size_t)j * elem_bytes, (const uint8_t*)src + chunk_elem(c, j, nf, per) * elem_bytes,
             (size_t)std::min<uint32_t>(c < nf ? kUnit : nc, nc - j) * elem_bytes);
    std::vector<uint8_t> plane;
    const bool split = split_plane && c < nf;
    encode_chunk(P, gathered.data(), nc, lanes, nw[c], np[c], chunks[c], split ? &plane : nullptr);
    if (split)
      for (uint64_t b = 0; b * pblk < plane.size(); ++b)
        memcpy(plane_region.data() + (b * nf + c) * pblk, plane.data() + b * pblk, pblk);
  });

  uint64_t total = preg + plane_region.size();
  std::vector<uint64_t> offs(nch);
  for (uint32_t c = 0; c < nch; ++c) { offs[c] = total; total += chunks[c].size(); }
  const uint64_t end = total;
  total = pad256(total);                             // blob lengths are multiples of 256
  if (total > cap) return BS_ERR_CAP;
  memset(dst, 0, preg);
  memcpy(dst, "BSCK", 4);
  dst[4] = kVersion; dst[5] = (uint8_t)elem_bytes; dst[6] = (uint8_t)P.mode; dst[7] = 12;
  put64(dst + 8, n); put32(dst + 16, steps); put16(dst + 20, lanes); put16(dst + 22, P.nsym);
  put32(dst + 24, nch); put32(dst + 28, 0);
  for (uint32_t s = 0; s < P.nsym; ++s)
    put32(dst + 32 + 4 * s, (P.value[s] & 0xFFFF) | (P.freq[s] << 16) | (P.consume[s] << 31));
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

}  // extern "C"
