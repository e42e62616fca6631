// CPU check of the GPU zstd decoder's core (bigsmall_amd/csrc/zstd_core.h),
// run as a one-lane team and, when built with BS_ZSTD_TEAM64, also as the GPU's
// 64-lane team (lanes as fibers, bigsmall_amd/csrc/simt_cpu.h), against
// libzstd (the format's reference implementation). Built by
// tests/test_zstd_core_cpu.py under AddressSanitizer and UBSan, so any read or
// write outside the input, output or literal buffers fails the run. The
// 64-lane team must give the one-lane team's error code and bytes on every
// frame: its lanes run one after another between barriers, so a lane that
// reads what another writes without a barrier between them is caught.
//   1. round trips: several data kinds x compression levels, checksum and
//      no-content-size frames, back-to-back frames with a skippable frame;
//   2. corruptions: single-bit flips, byte overwrites and truncations of
//      frames; every mutated frame must decode to what libzstd decodes it to,
//      or return an error (never decode where libzstd refuses).
// Prints one summary line; exit status 0 when every check holds.
#ifdef BS_ZSTD_TEAM64
#include "../../bigsmall_amd/csrc/simt_cpu.h"
#else
#define __host__
#define __device__
#define __forceinline__ inline
#endif
#include "../../bigsmall_amd/csrc/zstd_core.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

extern "C" {
size_t ZSTD_compressBound(size_t);
unsigned ZSTD_isError(size_t);
void* ZSTD_createCCtx(void);
size_t ZSTD_freeCCtx(void*);
size_t ZSTD_CCtx_setParameter(void*, int, int);
size_t ZSTD_compress2(void*, void*, size_t, const void*, size_t);
size_t ZSTD_decompress(void*, size_t, const void*, size_t);
}

namespace {

struct OneLane {
  static constexpr uint32_t size = 1;
  uint32_t lane() const { return 0; }
  void sync() const {}
};

using Bytes = std::vector<uint8_t>;

Bytes compress(const Bytes& in, int level, int checksum = 0, int content_size = 1) {
  Bytes out(ZSTD_compressBound(in.size()) + 16);
  void* c = ZSTD_createCCtx();
  ZSTD_CCtx_setParameter(c, 100, level);
  ZSTD_CCtx_setParameter(c, 200, content_size);
  ZSTD_CCtx_setParameter(c, 201, checksum);
  const size_t r = ZSTD_compress2(c, out.data(), out.size(), in.data(), in.size());
  ZSTD_freeCCtx(c);
  if (ZSTD_isError(r)) {
    std::puts("libzstd compression failed");
    std::exit(2);
  }
  out.resize(r);
  return out;
}

bs_zstd::ZState g_state;

#ifdef BS_ZSTD_TEAM64
// The GPU's team: 64 lanes, the workgroup barrier as sync().
struct FiberTeam {
  static constexpr uint32_t size = 64;
  uint32_t lane() const { return __lane_id(); }
  void sync() const { __syncthreads(); }
};
long g_team_mismatch = 0;
#endif

// Decodes `frame` (copied to an exact-size heap block) into an exact-size
// block of `cap` bytes; returns the error code, output in *out.
template <class Run>
int decode_with(const Bytes& frame, size_t cap, Bytes* out, Run run) {
  static Bytes lit(bs_zstd::kBlockMax);
  uint8_t* src = new uint8_t[frame.size() ? frame.size() : 1];
  if (!frame.empty()) std::memcpy(src, frame.data(), frame.size());
  uint8_t* dst = new uint8_t[cap ? cap : 1];
  uint64_t got = 0;
  int e = run(src, frame.size(), dst, cap, lit.data(), got);
  if (e == 0 && got != cap) e = bs_zstd::kErrOutput;
  out->assign(dst, dst + (e ? 0 : got));
  delete[] src;
  delete[] dst;
  return e;
}

int decode(const Bytes& frame, size_t cap, Bytes* out) {
  const int e = decode_with(frame, cap, out, [](const uint8_t* s, uint64_t n, uint8_t* d, uint64_t c, uint8_t* lit,
                                                 uint64_t& got) {
    return bs_zstd::zstd_frames(OneLane{}, g_state, s, n, d, c, lit, got);
  });
#ifdef BS_ZSTD_TEAM64
  Bytes out64;
  const int e64 = decode_with(frame, cap, &out64, [](const uint8_t* s, uint64_t n, uint8_t* d, uint64_t c,
                                                     uint8_t* lit, uint64_t& got) {
    int err = 0;
    bs_simt::launch([&] {
      __shared__ bs_zstd::ZState z;
      uint64_t g = 0;
      const int r = bs_zstd::zstd_frames(FiberTeam{}, z, s, n, d, c, lit, g);
      if (__lane_id() == 0) {
        err = r;
        got = g;
      }
    }, dim3(1), dim3(64), 0, nullptr);
    return err;
  });
  if (e64 != e || out64 != *out) ++g_team_mismatch;
#endif
  return e;
}

}  // namespace

int main(int argc, char** argv) {
  const int corruptions = argc > 1 ? std::atoi(argv[1]) : 600;
  std::mt19937_64 rng(1);
  std::vector<std::pair<std::string, Bytes>> data;
  for (size_t n : {1ul, 100ul, 4096ul, 200000ul}) {
    Bytes r(n), z(n, 0);
    for (auto& b : r) b = (uint8_t)rng();
    data.emplace_back("random" + std::to_string(n), r);
    data.emplace_back("zeros" + std::to_string(n), z);
  }
  for (size_t n : {4096ul, 300000ul}) {          // norm-weight indices: 16 values, skewed
    Bytes v(n);
    std::normal_distribution<double> g(0, 3);
    for (auto& b : v) {
      const int x = (int)std::lround(g(rng)) + 8;
      b = (uint8_t)(x < 0 ? 0 : x > 15 ? 15 : x);
    }
    data.emplace_back("lowcard" + std::to_string(n), v);
  }
  {
    Bytes v(400000);
    std::normal_distribution<float> g(0, 0.02f);
    for (size_t i = 0; i < v.size() / 2; ++i) {  // bf16 N(0, 0.02), round to nearest even
      const float f = g(rng);
      uint32_t u;
      std::memcpy(&u, &f, 4);
      const uint16_t h = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
      std::memcpy(&v[2 * i], &h, 2);
    }
    data.emplace_back("bf16", v);
  }
  {
    std::string s;
    while (s.size() < 300000) s += "the quick brown fox " + std::to_string(rng() % 1000) + " jumps\n";
    data.emplace_back("text", Bytes(s.begin(), s.end()));
  }
  long round_trips = 0, failures = 0;
  auto expect = [&](const char* what, const Bytes& frame, const Bytes& want) {
    Bytes got;
    ++round_trips;
    if (decode(frame, want.size(), &got) != 0 || got != want) {
      ++failures;
      std::printf("round trip failed: %s\n", what);
    }
  };
  for (auto& [name, v] : data)
    for (int level : {-5, 1, 3, 9, 19, 22}) expect((name + " level " + std::to_string(level)).c_str(),
                                                  compress(v, level), v);
  const Bytes& text = data.back().second;
  expect("checksum", compress(text, 3, 1), text);
  expect("no content size", compress(text, 19, 0, 0), text);
  {
    Bytes f = compress(data[0].second, 3), in = data[0].second;
    const uint8_t skip[12] = {0x50, 0x2A, 0x4D, 0x18, 4, 0, 0, 0, 1, 2, 3, 4};
    f.insert(f.end(), skip, skip + 12);
    const Bytes g = compress(text, 19);
    f.insert(f.end(), g.begin(), g.end());
    in.insert(in.end(), text.begin(), text.end());
    expect("back-to-back frames", f, in);
  }

  long same = 0, differ = 0, only_ours = 0, only_lib = 0, both_reject = 0;
  const char* sources[] = {"lowcard4096", "text", "bf16", "random4096"};
  for (const char* src_name : sources) {
    const Bytes* in = nullptr;
    for (auto& [name, v] : data)
      if (name == src_name) in = &v;
    for (int level : {1, 19}) {
      const Bytes f = compress(*in, level);
      for (int it = 0; it < corruptions; ++it) {
        Bytes g = f;
        if (it % 3 == 0) g[rng() % g.size()] ^= (uint8_t)(1u << (rng() % 8));
        else if (it % 3 == 1) g[rng() % g.size()] = (uint8_t)rng();
        else g.resize(rng() % g.size());
        Bytes ours;
        const int e = decode(g, in->size(), &ours);
        Bytes ref(in->size() + 1);
        const size_t r = ZSTD_decompress(ref.data(), in->size(), g.data(), g.size());
        const bool lib_ok = !ZSTD_isError(r) && r == in->size();
        if (e == 0 && lib_ok) (std::memcmp(ref.data(), ours.data(), r) == 0 ? same : differ)++;
        else if (e == 0) ++only_ours;
        else if (lib_ok) ++only_lib;
        else ++both_reject;
      }
    }
  }
  long team = 0;
#ifdef BS_ZSTD_TEAM64
  team = g_team_mismatch;
  std::printf("64-lane team differs from one lane on %ld frames\n", team);
#endif
  std::printf("round trips %ld (failed %ld); corruptions: decoded like libzstd %ld, decoded differently %ld, "
              "decoded where libzstd refuses %ld, refused where libzstd decodes %ld, both refuse %ld\n",
              round_trips, failures, same, differ, only_ours, only_lib, both_reject);
  return (failures || differ || only_ours || team) ? 1 : 0;
}
