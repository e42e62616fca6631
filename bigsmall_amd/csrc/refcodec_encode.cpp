// Host encoders of the reference's rANS-family bf16 formats, so compress()
// can write the containers the reference writes under its gpu_optimised and
// prefer_speed choices (bigsmall/codec_registry.py:316-391):
//   bf16_parallel_v1      bigsmall/codecs/bf16_parallel.py:77-135, 186-259
//                         (tables: rans.py:34-92; streams: rans.py:115-162)
//   bf16_se_tans          bigsmall/codecs/bf16_tans.py:46-55, 68-118
//                         (tables: numba_rans.py:45-85; streams: numba_rans.py:108-150)
//   bf16_se_single_kernel bigsmall/codecs/single_kernel.py:193-428
//                         (tables: single_kernel.py:53-110; streams: :121-156)
// The byte layouts are those formats' own (the decoders of any reader depend
// on them). Independent chains (the N streams of bf16_parallel_v1, the
// per-exponent mantissa buckets) are encoded on a small thread pool.
//
// Every format codes a bf16 word w as the sign+exponent symbol
// (w >> 15) << 8 | (w >> 7 & 0xFF) with M = 4096, and its 7-bit mantissa in
// the bucket of its exponent with M = 1024. rANS: 32-bit state starting at
// L = 2^16, symbols encoded last to first, a 16-bit word emitted while the
// state is at least (2^32 / M) * f; the stream is [u32 final state][u16 words
// in decode order].
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

#include "../../include/bigsmall_hip.h"

namespace {

constexpr uint32_t kL = 1u << 16;
constexpr int kSeAlphabet = 512;
constexpr int kMantAlphabet = 128;
constexpr uint32_t kMse = 4096;
constexpr uint32_t kMmant = 1024;

typedef std::vector<uint32_t> Freqs;

// rans.quantise_frequencies (rans.py:34-92; numba_rans.py:45-85 is the same
// rule): floor-scale to M, nonzero counts at least 1, then the difference to M
// spread one unit at a time over the symbols in stable descending order of
// their scaled frequency (wrapping), never taking a nonzero symbol below 1.
int quantise_ranked(const std::vector<int64_t>& counts, uint32_t M, Freqs& out) {
  const size_t A = counts.size();
  out.assign(A, 0);
  int64_t total = 0;
  size_t n_nz = 0;
  for (int64_t c : counts) {
    total += c;
    n_nz += c > 0;
  }
  if (n_nz == 0) {
    out[0] = M;
    return BS_OK;
  }
  if (n_nz > M) return BS_ERR_FORMAT;
  std::vector<int64_t> s(A, 0);
  int64_t sum = 0;
  for (size_t i = 0; i < A; ++i) {
    if (counts[i] > 0) s[i] = std::max<int64_t>(1, counts[i] * (int64_t)M / total);
    sum += s[i];
  }
  int64_t diff = (int64_t)M - sum;
  if (diff != 0) {
    std::vector<uint32_t> order(A);
    for (size_t i = 0; i < A; ++i) order[i] = (uint32_t)i;
    std::stable_sort(order.begin(), order.end(), [&](uint32_t a, uint32_t b) { return s[a] > s[b]; });
    size_t i = 0;
    if (diff > 0) {
      for (; diff > 0; --diff, ++i) s[order[i % A]] += 1;
    } else {
      while (diff < 0) {
        const uint32_t j = order[i % A];
        if (s[j] > 1) {
          s[j] -= 1;
          ++diff;
        }
        ++i;
        if (i > 100 * A) return BS_ERR_FORMAT;      // the reference raises here
      }
    }
  }
  for (size_t i = 0; i < A; ++i) out[i] = (uint32_t)s[i];
  return BS_OK;
}

// single_kernel._quantise_inplace (single_kernel.py:53-110): floor-scale with a
// minimum of 1, then add to / take from the first symbol holding the largest
// frequency, one unit at a time.
void quantise_argmax(const std::vector<int64_t>& counts, uint32_t M, Freqs& out) {
  const size_t A = counts.size();
  out.assign(A, 0);
  int64_t total = 0;
  size_t n_nz = 0;
  for (int64_t c : counts) {
    total += c;
    n_nz += c > 0;
  }
  if (n_nz == 0) {
    out[0] = M;
    return;
  }
  int64_t sum = 0;
  for (size_t i = 0; i < A; ++i) {
    if (counts[i] > 0) out[i] = (uint32_t)std::max<int64_t>(1, counts[i] * (int64_t)M / total);
    sum += out[i];
  }
  auto argmax = [&]() {
    size_t best = 0;
    uint32_t v = 0;
    for (size_t i = 0; i < A; ++i)
      if (out[i] > v) {
        v = out[i];
        best = i;
      }
    return best;
  };
  int64_t diff = (int64_t)M - sum;
  for (; diff > 0; --diff) out[argmax()] += 1;
  for (size_t guard = 0; diff < 0 && guard < 50 * A; ++guard) {
    const size_t b = argmax();
    if (out[b] <= 1) break;
    out[b] -= 1;
    ++diff;
  }
}

// One rANS chain. Symbols are read as sym(i) for i in [0, n).
struct Chain {
  uint32_t state = kL;
  std::vector<uint16_t> words;     // decode order
  size_t bytes() const { return 4 + 2 * words.size(); }
  void put(std::vector<uint8_t>& o) const {
    const size_t p = o.size();
    o.resize(p + bytes());
    memcpy(o.data() + p, &state, 4);
    if (!words.empty()) memcpy(o.data() + p + 4, words.data(), 2 * words.size());
  }
};

template <class Sym>
void rans_encode(size_t n, Sym sym, const Freqs& f, uint32_t M, Chain& c) {
  std::vector<uint32_t> cum(f.size() + 1, 0);
  for (size_t i = 0; i < f.size(); ++i) cum[i + 1] = cum[i] + f[i];
  const uint64_t per = (1ull << 32) / M;
  uint64_t x = kL;
  c.words.clear();
  c.words.reserve(n / 4 + 16);
  for (size_t i = n; i-- > 0;) {
    const uint32_t s = sym(i);
    const uint64_t fs = f[s];
    const uint64_t upper = per * fs;
    while (x >= upper) {
      c.words.push_back((uint16_t)(x & 0xFFFF));
      x >>= 16;
    }
    x = (x / fs) * M + cum[s] + (x % fs);
  }
  std::reverse(c.words.begin(), c.words.end());
  c.state = (uint32_t)x;
}

// Runs jobs [0, n) on up to `threads` threads.
template <class F>
void parallel_for(size_t n, int threads, F fn) {
  const size_t t = std::max<size_t>(1, std::min<size_t>((size_t)std::max(1, threads), n));
  if (t == 1) {
    for (size_t i = 0; i < n; ++i) fn(i);
    return;
  }
  std::atomic<size_t> next{0};
  std::vector<std::thread> pool;
  for (size_t k = 0; k < t; ++k)
    pool.emplace_back([&] {
      for (size_t i = next++; i < n; i = next++) fn(i);
    });
  for (auto& th : pool) th.join();
}

struct Out {
  std::vector<uint8_t> b;
  void u8(uint32_t v) { b.push_back((uint8_t)v); }
  void u16(uint32_t v) { u8(v & 0xFF); u8(v >> 8); }
  void u32(uint32_t v) { u16(v & 0xFFFF); u16(v >> 16); }
  void raw(const void* p, size_t n) { b.insert(b.end(), (const uint8_t*)p, (const uint8_t*)p + n); }
};

inline uint32_t se_of(uint16_t w) { return ((uint32_t)(w >> 15) << 8) | ((w >> 7) & 0xFFu); }
inline uint32_t exp_of(uint16_t w) { return (w >> 7) & 0xFFu; }
inline uint32_t mant_of(uint16_t w) { return w & 0x7Fu; }

// Stable counting sort of element indices by exponent: order[] lists the
// elements of `idx(0..n)` bucket by bucket, bstart[e] where bucket e begins.
template <class Idx>
void sort_by_exp(const uint16_t* w, size_t n, Idx idx, std::vector<uint32_t>& order, std::vector<uint64_t>& bstart) {
  bstart.assign(257, 0);
  for (size_t i = 0; i < n; ++i) ++bstart[exp_of(w[idx(i)]) + 1];
  for (int e = 0; e < 256; ++e) bstart[e + 1] += bstart[e];
  std::vector<uint64_t> cur(bstart.begin(), bstart.end() - 1);
  order.resize(n);
  for (size_t i = 0; i < n; ++i) order[cur[exp_of(w[idx(i)])]++] = (uint32_t)idx(i);
}

// Shared tables of bf16_parallel_v1 (bf16_parallel.py:77-103).
int par1_encode(const uint16_t* w, uint64_t n, uint32_t n_streams, int threads, Out& out) {
  const uint32_t N = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(n_streams, n));
  std::vector<int64_t> se_counts(kSeAlphabet, 0), exp_counts(256, 0);
  std::vector<std::vector<int64_t>> mant_counts(256, std::vector<int64_t>(kMantAlphabet, 0));
  for (uint64_t i = 0; i < n; ++i) {
    ++se_counts[se_of(w[i])];
    ++exp_counts[exp_of(w[i])];
    ++mant_counts[exp_of(w[i])][mant_of(w[i])];
  }
  Freqs se_f;
  if (quantise_ranked(se_counts, kMse, se_f) != BS_OK) return BS_ERR_FORMAT;
  std::vector<Freqs> mant_f(256);
  std::vector<uint32_t> exps;
  for (int e = 0; e < 256; ++e)
    if (exp_counts[e] > 0) {
      exps.push_back((uint32_t)e);
      if (quantise_ranked(mant_counts[e], kMmant, mant_f[e]) != BS_OK) return BS_ERR_FORMAT;
    }
  // header (bf16_parallel.py:106-135)
  out.raw("PAR1", 4);
  out.u32((uint32_t)n);
  out.u16(N);
  out.u16(12);
  out.u16(10);
  uint32_t n_se_nz = 0;
  for (uint32_t f : se_f) n_se_nz += f > 0;
  out.u16(n_se_nz);
  for (int s = 0; s < kSeAlphabet; ++s)
    if (se_f[s]) out.u16((uint32_t)s);
  for (int s = 0; s < kSeAlphabet; ++s)
    if (se_f[s]) out.u32(se_f[s]);
  out.u32((uint32_t)exps.size());
  for (uint32_t e : exps) out.u16(e);
  for (uint32_t e : exps) {
    uint32_t k = 0;
    for (uint32_t f : mant_f[e]) k += f > 0;
    out.u8(k);
    for (int m = 0; m < kMantAlphabet; ++m)
      if (mant_f[e][m]) out.u8((uint32_t)m);
    for (int m = 0; m < kMantAlphabet; ++m)
      if (mant_f[e][m]) out.u32(mant_f[e][m]);
  }
  // streams: elements k, k+N, ... (bf16_parallel.py:205-244), one job each
  std::vector<Out> sb(N);
  parallel_for(N, threads, [&](size_t k) {
    const uint64_t nk = (n - 1 - k) / N + 1;
    auto idx = [&](size_t i) { return (uint64_t)k + (uint64_t)i * N; };
    Out& o = sb[k];
    Chain se;
    rans_encode(nk, [&](size_t i) { return se_of(w[idx(i)]); }, se_f, kMse, se);
    o.u32((uint32_t)se.bytes());
    se.put(o.b);
    std::vector<uint32_t> order;
    std::vector<uint64_t> bstart;
    sort_by_exp(w, nk, idx, order, bstart);
    std::vector<uint32_t> sexps;
    for (int e = 0; e < 256; ++e)
      if (bstart[e + 1] > bstart[e]) sexps.push_back((uint32_t)e);
    o.u32((uint32_t)sexps.size());
    for (uint32_t e : sexps) o.u16(e);
    for (uint32_t e : sexps) {
      const uint64_t b0 = bstart[e], cnt = bstart[e + 1] - b0;
      Chain m;
      rans_encode(cnt, [&](size_t i) { return mant_of(w[order[b0 + i]]); }, mant_f[e], kMmant, m);
      o.u32((uint32_t)cnt);
      o.u32((uint32_t)m.bytes());
      m.put(o.b);
    }
  });
  uint64_t off = 0;
  for (uint32_t k = 0; k < N; ++k) {
    out.u32((uint32_t)off);
    off += sb[k].b.size();
  }
  if (off > 0xFFFFFFFFull) return BS_ERR_ARG;
  out.u32((uint32_t)off);
  for (uint32_t k = 0; k < N; ++k) out.raw(sb[k].b.data(), sb[k].b.size());
  return BS_OK;
}

// bf16_se_tans (bf16_tans.py:68-118): one sign+exponent chain, then the
// tensor-wide mantissa buckets, each with its own table.
int tans_encode(const uint16_t* w, uint64_t n, int threads, Out& out) {
  std::vector<int64_t> se_counts(kSeAlphabet, 0);
  for (uint64_t i = 0; i < n; ++i) ++se_counts[se_of(w[i])];
  Freqs se_f;
  if (quantise_ranked(se_counts, kMse, se_f) != BS_OK) return BS_ERR_FORMAT;
  std::vector<uint32_t> order;
  std::vector<uint64_t> bstart;
  sort_by_exp(w, n, [](size_t i) { return (uint64_t)i; }, order, bstart);
  std::vector<uint32_t> exps;
  for (int e = 0; e < 256; ++e)
    if (bstart[e + 1] > bstart[e]) exps.push_back((uint32_t)e);
  // job 0: the sign+exponent chain; job 1 + b: bucket b
  Chain se;
  std::vector<Chain> mc(exps.size());
  std::vector<Freqs> mf(exps.size());
  std::atomic<int> err{BS_OK};
  parallel_for(1 + exps.size(), threads, [&](size_t j) {
    if (j == 0) {
      rans_encode(n, [&](size_t i) { return se_of(w[i]); }, se_f, kMse, se);
      return;
    }
    const uint32_t e = exps[j - 1];
    const uint64_t b0 = bstart[e], cnt = bstart[e + 1] - b0;
    std::vector<int64_t> c(kMantAlphabet, 0);
    for (uint64_t i = 0; i < cnt; ++i) ++c[mant_of(w[order[b0 + i]])];
    if (quantise_ranked(c, kMmant, mf[j - 1]) != BS_OK) {
      err = BS_ERR_FORMAT;
      return;
    }
    rans_encode(cnt, [&](size_t i) { return mant_of(w[order[b0 + i]]); }, mf[j - 1], kMmant, mc[j - 1]);
  });
  if (err != BS_OK) return err;
  Out m;
  m.u32((uint32_t)exps.size());
  for (uint32_t e : exps) m.u16(e);
  for (size_t b = 0; b < exps.size(); ++b) {
    const uint32_t e = exps[b];
    m.u32((uint32_t)(bstart[e + 1] - bstart[e]));
    uint32_t k = 0;
    for (uint32_t f : mf[b]) k += f > 0;
    m.u8(k);
    for (int s = 0; s < kMantAlphabet; ++s)
      if (mf[b][s]) m.u8((uint32_t)s);
    for (int s = 0; s < kMantAlphabet; ++s)
      if (mf[b][s]) m.u32(mf[b][s]);
    m.u32((uint32_t)mc[b].bytes());
    mc[b].put(m.b);
  }
  out.u32((uint32_t)n);
  uint32_t n_se_nz = 0;
  for (uint32_t f : se_f) n_se_nz += f > 0;
  out.u16(n_se_nz);
  for (int s = 0; s < kSeAlphabet; ++s)
    if (se_f[s]) out.u16((uint32_t)s);
  for (int s = 0; s < kSeAlphabet; ++s)
    if (se_f[s]) out.u32(se_f[s]);
  out.u32((uint32_t)se.bytes());
  se.put(out.b);
  out.u32((uint32_t)m.b.size());
  out.raw(m.b.data(), m.b.size());
  return BS_OK;
}

// bf16_se_single_kernel (single_kernel.py:193-428): the same two-level model
// with the argmax quantiser and explicit state / word-count fields.
int sk_encode(const uint16_t* w, uint64_t n, int threads, Out& out) {
  std::vector<int64_t> se_counts(kSeAlphabet, 0);
  for (uint64_t i = 0; i < n; ++i) ++se_counts[se_of(w[i])];
  Freqs se_f;
  quantise_argmax(se_counts, kMse, se_f);
  std::vector<uint32_t> order;
  std::vector<uint64_t> bstart;
  sort_by_exp(w, n, [](size_t i) { return (uint64_t)i; }, order, bstart);
  std::vector<uint32_t> exps;
  for (int e = 0; e < 256; ++e)
    if (bstart[e + 1] > bstart[e]) exps.push_back((uint32_t)e);
  Chain se;
  std::vector<Chain> mc(exps.size());
  std::vector<Freqs> mf(exps.size());
  parallel_for(1 + exps.size(), threads, [&](size_t j) {
    if (j == 0) {
      rans_encode(n, [&](size_t i) { return se_of(w[i]); }, se_f, kMse, se);
      return;
    }
    const uint32_t e = exps[j - 1];
    const uint64_t b0 = bstart[e], cnt = bstart[e + 1] - b0;
    std::vector<int64_t> c(kMantAlphabet, 0);
    for (uint64_t i = 0; i < cnt; ++i) ++c[mant_of(w[order[b0 + i]])];
    quantise_argmax(c, kMmant, mf[j - 1]);
    rans_encode(cnt, [&](size_t i) { return mant_of(w[order[b0 + i]]); }, mf[j - 1], kMmant, mc[j - 1]);
  });
  out.u32((uint32_t)n);
  uint32_t n_se_nz = 0;
  for (uint32_t f : se_f) n_se_nz += f > 0;
  out.u16(n_se_nz);
  for (int s = 0; s < kSeAlphabet; ++s)
    if (se_f[s]) out.u16((uint32_t)s);
  for (int s = 0; s < kSeAlphabet; ++s)
    if (se_f[s]) out.u32(se_f[s]);
  out.u32(se.state);
  out.u32((uint32_t)se.words.size());
  out.raw(se.words.data(), 2 * se.words.size());
  out.u32((uint32_t)exps.size());
  for (size_t b = 0; b < exps.size(); ++b) {
    const uint32_t e = exps[b];
    out.u16(e);
    uint32_t k = 0;
    for (uint32_t f : mf[b]) k += f > 0;
    out.u8(k);
    for (int s = 0; s < kMantAlphabet; ++s)
      if (mf[b][s]) out.u8((uint32_t)s);
    for (int s = 0; s < kMantAlphabet; ++s)
      if (mf[b][s]) out.u32(mf[b][s]);
    out.u32(mc[b].state);
    out.u32((uint32_t)(bstart[e + 1] - bstart[e]));
    out.u32((uint32_t)mc[b].words.size());
    out.raw(mc[b].words.data(), 2 * mc[b].words.size());
  }
  return BS_OK;
}

}  // namespace

extern "C" {

uint64_t bs_refcodec_encode_bound(int32_t codec, uint64_t n, uint32_t n_streams) {
  // <= one 16-bit word per symbol and two symbols per element; the tables of
  // 512 sign+exponent and 256 x 128 mantissa symbols; per stream of
  // bf16_parallel_v1 its lengths, exponent list and bucket fields
  const uint64_t tables = 16 + kSeAlphabet * 6 + 4 + 256 * 2 + 256 * (1 + kMantAlphabet * 5);
  const uint64_t buckets = 4 + 256 * 2 + 256 * (16 + 1 + kMantAlphabet * 5);
  const uint64_t ns = std::max<uint64_t>(1, std::min<uint64_t>(n_streams, n));   // the encoder's clamp
  const uint64_t streams = codec == BS_REF_PARALLEL ? (ns + 1) * (4 + 12 + buckets) : 12 + buckets;
  return 4 * n + tables + streams + 64;
}

int bs_refcodec_encode(int32_t codec, const uint16_t* h_src, uint64_t n, uint32_t n_streams, uint8_t* h_dst,
                       uint64_t cap, uint64_t* out_len, int n_threads) {
  if (!out_len || (n && !h_src) || codec < BS_REF_PARALLEL || codec > BS_REF_SINGLE_KERNEL) return BS_ERR_ARG;
  if (n > 0xFFFFFFFFull) return BS_ERR_ARG;
  *out_len = 0;
  if (n == 0) return BS_OK;               // an empty tensor is an empty blob in all three formats
  // N = max(1, min(n_streams, n)) (bigsmall/codecs/bf16_parallel.py:195); the
  // header stores N as a u16 (struct '<H'), so only a clamped N above 65535 fails
  if (codec == BS_REF_PARALLEL) {
    n_streams = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(n_streams, n));
    if (n_streams > 0xFFFF) return BS_ERR_ARG;
  }
  Out out;
  int rc = codec == BS_REF_PARALLEL ? par1_encode(h_src, n, n_streams, n_threads, out)
           : codec == BS_REF_TANS   ? tans_encode(h_src, n, n_threads, out)
                                    : sk_encode(h_src, n, n_threads, out);
  if (rc != BS_OK) return rc;
  *out_len = out.b.size();
  if (out.b.size() > cap || (!h_dst && cap)) return BS_ERR_CAP;
  if (cap) memcpy(h_dst, out.b.data(), out.b.size());
  return BS_OK;
}

}  // extern "C"
