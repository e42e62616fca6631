// CPU runs of the GPU decode kernels (bigsmall_amd/csrc/bsck_decode.hip,
// refcodec_decode.hip), built as host C++ with the SIMT emulation of
// bigsmall_amd/csrc/simt_cpu.h under AddressSanitizer and UBSan
// (tests/test_decode_cores_cpu.py builds and drives it).
//
// Input: a case file written by the test. Each case is a BSCK blob, or a
// reference-format blob with the stream descriptors and decode tables the
// library's host parser (bigsmall_amd/codecs/_refstreams.py) made from it
// (word arrays as blob offsets). Clean cases must decode to their expected
// bytes with a zero status word; corrupted cases may decode to anything or
// report a status, but every access must stay inside its buffers, which
// are allocated at their exact sizes so that the sanitizer sees any overrun.
// The clean BSCK blobs are then decoded again in batched launches.
// Prints a batch line and a summary line; exit status 0 when every clean
// case decoded right, alone and batched.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>

#include <vector>

#include "bigsmall_hip.h"

namespace {

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  template <class T>
  T get() {
    T v;
    if (p + sizeof(T) > end) {
      fprintf(stderr, "case file truncated\n");
      exit(3);
    }
    memcpy(&v, p, sizeof(T));
    p += sizeof(T);
    return v;
  }
  const uint8_t* take(uint64_t n) {
    if (n > (uint64_t)(end - p)) {
      fprintf(stderr, "case file truncated\n");
      exit(3);
    }
    const uint8_t* r = p;
    p += n;
    return r;
  }
};

// A buffer of exactly n bytes at a 256-byte aligned address (aligned_alloc
// sizes must be multiples of the alignment: the slack is poisoned by
// allocating it separately is not possible, so n is what the sanitizer
// guards when n is a multiple of 256; other sizes use malloc's 16-byte
// alignment, which every kernel access here needs at most).
struct Buf {
  uint8_t* p = nullptr;
  explicit Buf(uint64_t n, bool align256 = false) {
    if (align256) p = (uint8_t*)aligned_alloc(256, ((n + 255) / 256) * 256 + 256);
    else p = (uint8_t*)malloc(n ? n : 1);
    if (!p) exit(4);
  }
  ~Buf() { free(p); }
  Buf(const Buf&) = delete;
};

// Buffers for the batched launches, carved from one mapping that straddles
// an address whose low 32 bits cross 2^31: the first buffers have bit 31 of
// the low half clear, the later ones set. A 4 GiB + n reservation always
// holds such an address; only the n bytes around it are made accessible.
struct Pool {
  uint8_t* res = nullptr;
  uint8_t* base = nullptr;
  uint64_t res_size = 0, size = 0, used = 0;
  explicit Pool(uint64_t n) : size(n) {
    res_size = (4ull << 30) + 2 * n;
    void* m = mmap(nullptr, res_size, PROT_NONE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    if (m == MAP_FAILED) exit(4);
    res = (uint8_t*)m;
    const uintptr_t lo = (uintptr_t)res + n;                       // room below the crossing
    const uintptr_t cross = (lo & ~0xFFFFFFFFull) | 0x80000000ull;
    const uintptr_t at = (cross >= lo ? cross : cross + (1ull << 32)) - (256u << 10);   // 256 KiB below it
    base = (uint8_t*)at;
    if (mprotect(base, n, PROT_READ | PROT_WRITE) != 0) exit(4);
  }
  ~Pool() { munmap(res, res_size); }
  uint8_t* take(uint64_t n) {
    used = (used + 255) & ~255ull;
    if (used + n > size) exit(4);
    uint8_t* r = base + used;
    used += n ? n : 1;
    return r;
  }
};

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  FILE* f = fopen(argv[1], "rb");
  if (!f) return 2;
  std::vector<uint8_t> file;
  uint8_t tmp[1 << 16];
  size_t got;
  while ((got = fread(tmp, 1, sizeof tmp, f)) > 0) file.insert(file.end(), tmp, tmp + got);
  fclose(f);
  Reader r{file.data(), file.data() + file.size()};
  if (r.get<uint32_t>() != 0x5A465342u) return 2;   // "BSFZ"
  const uint32_t n_cases = r.get<uint32_t>();
  uint64_t clean_ok = 0, clean_bad = 0, refused_host = 0, flagged = 0, decoded = 0, scalar_mismatch = 0;
  struct Clean {
    std::vector<uint8_t> blob, want;
    uint64_t n;
    uint32_t eb;
  };
  std::vector<Clean> clean_bsck;   // decoded again together, through the batched entry point
  struct CleanRef {                 // a clean wave-serial case, as read (word arrays blob-relative)
    std::vector<uint8_t> blob, se, se_table, bstart, mb, tables, want;
    uint32_t ns, nb, nt;
    uint64_t n;
  };
  std::vector<CleanRef> clean_ref;  // decoded again together, with gaps between the tasks' SE groups
  CleanRef pending;
  for (uint32_t c = 0; c < n_cases; ++c) {
    const uint8_t kind = r.get<uint8_t>(), clean = r.get<uint8_t>();
    r.get<uint16_t>();
    const uint64_t n_out = r.get<uint64_t>();
    const uint32_t eb = r.get<uint32_t>();
    const uint64_t blob_len = r.get<uint64_t>();
    const uint8_t* blob_src = r.take(blob_len);
    Buf blob(blob_len);
    memcpy(blob.p, blob_src, blob_len);
    Buf out(n_out * eb);
    memset(out.p, 0x5A, n_out * eb);
    int32_t status = 0;
    int rc = BS_OK;
    if (kind == 0) {   // BSCK: the kernel reads the blob's own header
      bs_chunk_info info;
      rc = bs_chunk_inspect(blob.p, blob_len, &info);
      if (rc == BS_OK) rc = bs_chunk_decode(blob.p, blob_len, out.p, n_out, info.n_chunks, info.plane_mode, &status, nullptr);
    } else {           // reference formats: descriptors with blob-relative word arrays
      const uint32_t ns = r.get<uint32_t>(), nb = r.get<uint32_t>(), nt = r.get<uint32_t>();
      const uint32_t se_bytes = r.get<uint32_t>();   // 4096 pairs, and the 4-byte form when the tensor has it
      std::vector<bs_se_stream> se(ns);
      memcpy(se.data(), r.take((uint64_t)ns * sizeof(bs_se_stream)), (uint64_t)ns * sizeof(bs_se_stream));
      if (se_bytes != 4096 * 8 && se_bytes != 4096 * 8 + (4096 + 256) * 4) return 2;
      Buf se_table(se_bytes);
      memcpy(se_table.p, r.take(se_bytes), se_bytes);
      Buf bstart((uint64_t)ns * 257 * 4);
      memcpy(bstart.p, r.take((uint64_t)ns * 257 * 4), (uint64_t)ns * 257 * 4);
      std::vector<bs_mant_bucket> mb(nb);
      memcpy(mb.data(), r.take((uint64_t)nb * sizeof(bs_mant_bucket)), (uint64_t)nb * sizeof(bs_mant_bucket));
      Buf tables((uint64_t)nt * 4096);
      memcpy(tables.p, r.take((uint64_t)nt * 4096), (uint64_t)nt * 4096);
      if (clean && kind == 1) {
        auto bytes = [](const void* q, uint64_t n) {
          return std::vector<uint8_t>((const uint8_t*)q, (const uint8_t*)q + n);
        };
        pending = CleanRef{bytes(blob.p, blob_len), bytes(se.data(), (uint64_t)ns * sizeof(bs_se_stream)),
                           bytes(se_table.p, se_bytes), bytes(bstart.p, (uint64_t)ns * 257 * 4),
                           bytes(mb.data(), (uint64_t)nb * sizeof(bs_mant_bucket)), bytes(tables.p, (uint64_t)nt * 4096),
                           {}, ns, nb, nt, n_out};
      }
      for (auto& s : se) s.words = blob.p + (uintptr_t)s.words;
      for (auto& b : mb) b.words = blob.p + (uintptr_t)b.words;
      Buf d_se(ns * sizeof(bs_se_stream)), d_mb(nb * sizeof(bs_mant_bucket));
      memcpy(d_se.p, se.data(), ns * sizeof(bs_se_stream));
      memcpy(d_mb.p, mb.data(), nb * sizeof(bs_mant_bucket));
      if (kind == 1) {
        const uint64_t wb = bs_refcodec_serial_work_bytes(n_out, ns);
        Buf work(wb, true);
        rc = bs_refcodec_decode_serial((const bs_se_stream*)d_se.p, ns, (const uint32_t*)se_table.p,
                                       (const uint32_t*)bstart.p, (const bs_mant_bucket*)d_mb.p, nb,
                                       (const uint32_t*)tables.p, nt, (uint16_t*)out.p, n_out, work.p, wb, &status,
                                       nullptr);
        // the same decode as a one-task batch whose chains read 4-byte tables
        // through the scalar path (the SE chains only when the table has that
        // form); its output and status must be the same
        if (rc == BS_OK && n_out > 0 && n_out <= 0xFFFFFFFFull) {
          Buf out2(n_out * eb), work2(wb, true);
          memset(out2.p, 0x5A, n_out * eb);
          const uint32_t per = bs_refcodec_serial_chains_per_group();
          bs_ref_task t{};
          t.streams = (const bs_se_stream*)d_se.p;
          t.se_table = (const uint32_t*)se_table.p;
          t.bstart = (const uint32_t*)bstart.p;
          t.buckets = (const bs_mant_bucket*)d_mb.p;
          t.mant_tables = (const uint32_t*)tables.p;
          t.out = (uint16_t*)out2.p;
          t.n_out = n_out;
          t.n_streams = ns;
          t.n_buckets = nb;
          t.n_tables = nt;
          t.flags = BS_REF_FLAG_MANT_SCALAR | (se_bytes > 4096 * 8 ? BS_REF_FLAG_SE_SCALAR : 0u);
          const uint32_t se_g = (ns + per - 1) / per, mant_g = (nb + per - 1) / per;
          const uint32_t tiles = bs_refcodec_serial_tiles(n_out, ns);
          Buf d_task(sizeof t);
          memcpy(d_task.p, &t, sizeof t);
          int32_t status2 = 0;
          const int rc2 = bs_refcodec_decode_serial_batch((const bs_ref_task*)d_task.p, 1, se_g, mant_g, ns * tiles, ns,
                                                          work2.p, wb, &status2, nullptr);
          if (rc2 != rc || status2 != status || (status == 0 && memcmp(out.p, out2.p, n_out * eb) != 0)) {
            ++scalar_mismatch;
            fprintf(stderr, "case %u: scalar-table batch rc %d status 0x%x, single rc %d status 0x%x\n", c, rc2,
                    status2, rc, status);
          }
        }
      } else {
        Buf perm(n_out * 4);
        rc = bs_refcodec_decode((const bs_se_stream*)d_se.p, ns, (const uint32_t*)se_table.p, (const uint32_t*)bstart.p,
                                (const bs_mant_bucket*)d_mb.p, nb, (const uint32_t*)tables.p, nt, (uint16_t*)out.p,
                                n_out, (uint32_t*)perm.p, &status, nullptr);
      }
    }
    const uint8_t* want = clean ? r.take(n_out * eb) : nullptr;
    if (clean && kind == 0)
      clean_bsck.push_back({std::vector<uint8_t>(blob_src, blob_src + blob_len),
                            std::vector<uint8_t>(want, want + n_out * eb), n_out, eb});
    if (clean && kind == 1 && n_out > 0) {
      pending.want.assign(want, want + n_out * eb);
      clean_ref.push_back(std::move(pending));
    }
    if (clean) {
      if (rc == BS_OK && status == 0 && memcmp(out.p, want, n_out * eb) == 0) {
        ++clean_ok;
      } else {
        ++clean_bad;
        fprintf(stderr, "clean case %u (kind %u, n %llu): rc %d status 0x%x\n", c, kind, (unsigned long long)n_out,
                rc, status);
      }
    } else if (rc != BS_OK) {
      ++refused_host;
    } else if (status != 0) {
      ++flagged;
    } else {
      ++decoded;
    }
  }
  // Batched launches of the clean BSCK blobs: once as they are (up to 64
  // tasks: the task lookup's last round alone), five times over (one
  // narrowing round of the wavefront vote first) and, for the blobs of at
  // most 256 elements, 4,096, 4,097 and 4,200 tasks: 4,096 is the most that
  // one narrowing round leaves at 64 (two dependent loads), 4,097 and more
  // take two narrowing rounds (three loads). Some buffers sit at addresses
  // with bit 31 of the low half set, so a lookup that widened that half with
  // sign extension would decode from a wrong address.
  uint64_t batch_ok = 0, batch_bad = 0, high_bit = 0;
  std::vector<size_t> small;
  for (size_t i = 0; i < clean_bsck.size(); ++i)
    if (clean_bsck[i].n <= 256) small.push_back(i);
  std::vector<std::vector<size_t>> plans(5);
  for (size_t i = 0; i < clean_bsck.size(); ++i) plans[0].push_back(i);
  for (int r = 0; r < 5; ++r) plans[1].insert(plans[1].end(), plans[0].begin(), plans[0].end());
  const size_t big[3] = {4096, 4097, 4200};
  for (int k = 0; k < 3; ++k)
    for (size_t t = 0; !small.empty() && t < big[k]; ++t) plans[2 + k].push_back(small[t % small.size()]);
  for (const auto& plan : plans) {
    const size_t nt = plan.size();
    if (nt == 0) continue;
    Pool pool(64ull << 20);
    std::vector<uint8_t*> blobs, outs;
    std::vector<bs_chunk_task> tasks(nt);
    uint32_t groups = 0, max_mode = 0;
    const uint32_t per_group = (uint32_t)bs_chunk_chunks_per_group();
    for (size_t t = 0; t < nt; ++t) {
      const Clean& c = clean_bsck[plan[t]];
      blobs.push_back(pool.take(c.blob.size()));
      memcpy(blobs.back(), c.blob.data(), c.blob.size());
      outs.push_back(pool.take(c.n * c.eb));
      memset(outs.back(), 0x5A, c.n * c.eb);
      bs_chunk_info info;
      if (bs_chunk_inspect(blobs.back(), c.blob.size(), &info) != BS_OK) return 5;
      tasks[t] = bs_chunk_task{blobs.back(), c.blob.size(), outs.back(), c.n, groups, info.n_chunks};
      groups += (info.n_chunks + per_group - 1) / per_group;
      if (info.plane_mode > max_mode) max_mode = info.plane_mode;
      high_bit += (((uintptr_t)blobs.back() >> 31) & 1u) + (((uintptr_t)outs.back() >> 31) & 1u);
    }
    Buf d_tasks(nt * sizeof(bs_chunk_task));
    memcpy(d_tasks.p, tasks.data(), nt * sizeof(bs_chunk_task));
    int32_t status = 0;
    const int rc = bs_chunk_decode_batch((const bs_chunk_task*)d_tasks.p, (uint32_t)nt, groups, max_mode, &status,
                                         nullptr);
    for (size_t t = 0; t < nt; ++t) {
      const Clean& c = clean_bsck[plan[t]];
      if (rc == BS_OK && status == 0 && memcmp(outs[t], c.want.data(), c.n * c.eb) == 0) {
        ++batch_ok;
      } else {
        ++batch_bad;
        ++clean_bad;
        fprintf(stderr, "batch of %zu, task %zu (n %llu): rc %d status 0x%x\n", nt, t, (unsigned long long)c.n, rc,
                status);
      }
    }
  }
  // A task table out of order whose lookup lands on an empty task (a blob
  // whose header reads n = 0, no chunks): the workgroup must stop at the
  // header check, flag it and read nothing past the blob. Tasks: a clean blob
  // at wg_begin 0, the empty one at 5, the clean blob again at 1, so
  // workgroup 1 counts two tasks at or before it and takes the second.
  uint64_t empty_flagged = 0;
  if (!clean_bsck.empty()) {
    const Clean& c = clean_bsck[0];
    Buf b0(c.blob.size()), b1(c.blob.size()), o0(c.n * c.eb), o1(c.n * c.eb), e(256), eo(16);
    memcpy(b0.p, c.blob.data(), c.blob.size());
    memcpy(b1.p, c.blob.data(), c.blob.size());
    memset(e.p, 0, 256);
    memcpy(e.p, "BSCK", 4);
    e.p[4] = 3; e.p[5] = 2; e.p[6] = 1; e.p[7] = 12;    // version, bf16, dense plane, 12-bit precision
    e.p[16] = 16; e.p[20] = 128; e.p[22] = 1;            // 16 steps, 128 lanes, one symbol; n = 0, no chunks
    const uint32_t sym = (0x7Fu << 7) | (4096u << 16) | (1u << 31);
    memcpy(e.p + 32, &sym, 4);
    bs_chunk_info info;
    if (bs_chunk_inspect(b0.p, c.blob.size(), &info) != BS_OK) return 5;
    const uint32_t g = (info.n_chunks + (uint32_t)bs_chunk_chunks_per_group() - 1) / (uint32_t)bs_chunk_chunks_per_group();
    bs_chunk_task tasks[3] = {{b0.p, c.blob.size(), o0.p, c.n, 0u, info.n_chunks},
                              {e.p, 256u, eo.p, 0u, 5u, 0u},
                              {b1.p, c.blob.size(), o1.p, c.n, 1u, info.n_chunks}};
    Buf d_tasks(sizeof tasks);
    memcpy(d_tasks.p, tasks, sizeof tasks);
    int32_t status = 0;
    const int rc = bs_chunk_decode_batch((const bs_chunk_task*)d_tasks.p, 3u, 1u + g, info.plane_mode, &status, nullptr);
    if (rc == BS_OK && (status & BS_DEV_ERR_HEADER)) empty_flagged = 1;
    else {
      ++clean_bad;
      fprintf(stderr, "out-of-order table with an empty task: rc %d status 0x%x\n", rc, status);
    }
  }
  // The clean wave-serial cases (up to 8) in one batched launch whose SE
  // groups have gaps: task i's groups start at i * C, C one more than the
  // most groups of any task, in a grid of 8C SE slots (the layout that puts
  // each task on an XCD of its own), every other task with its SE table read
  // through the scalar path where it has that form. Each must decode to its
  // source.
  uint64_t ref_batch_ok = 0;
  if (!clean_ref.empty()) {
    const size_t nt = clean_ref.size() < 8 ? clean_ref.size() : 8;
    const uint32_t per = bs_refcodec_serial_chains_per_group();
    uint32_t C = 0;
    for (size_t i = 0; i < nt; ++i) {
      const uint32_t g = (clean_ref[i].ns + per - 1) / per;
      if (g > C) C = g;
    }
    C += 1;
    std::vector<Buf*> keep;
    auto copy = [&](const std::vector<uint8_t>& v) {
      keep.push_back(new Buf(v.size() ? v.size() : 1));
      if (!v.empty()) memcpy(keep.back()->p, v.data(), v.size());
      return keep.back()->p;
    };
    std::vector<bs_ref_task> tasks(nt);
    std::vector<uint8_t*> outs(nt);
    uint32_t mant_g = 0, tiles = 0, streams = 0;
    uint64_t work = 0;
    for (size_t i = 0; i < nt; ++i) {
      CleanRef& c = clean_ref[i];
      uint8_t* blob = copy(c.blob);
      std::vector<bs_se_stream> se(c.ns);
      std::vector<bs_mant_bucket> mb(c.nb);
      memcpy(se.data(), c.se.data(), c.se.size());
      memcpy(mb.data(), c.mb.data(), c.mb.size());
      for (auto& q : se) q.words = blob + (uintptr_t)q.words;
      for (auto& q : mb) q.words = blob + (uintptr_t)q.words;
      bs_ref_task& t = tasks[i];
      t.streams = (const bs_se_stream*)copy(std::vector<uint8_t>((uint8_t*)se.data(), (uint8_t*)se.data() + c.se.size()));
      t.se_table = (const uint32_t*)copy(c.se_table);
      t.bstart = (const uint32_t*)copy(c.bstart);
      t.buckets = (const bs_mant_bucket*)copy(std::vector<uint8_t>((uint8_t*)mb.data(), (uint8_t*)mb.data() + c.mb.size()));
      t.mant_tables = (const uint32_t*)copy(c.tables);
      outs[i] = copy(std::vector<uint8_t>(c.n * 2, 0x5A));
      t.out = (uint16_t*)outs[i];
      t.n_out = c.n;
      t.work_offset = work;
      t.n_streams = c.ns;
      t.n_buckets = c.nb;
      t.n_tables = c.nt;
      t.se_group_begin = (uint32_t)i * C;
      t.tile_begin = tiles;
      t.stream_begin = streams;
      t.mant_group_begin = mant_g;
      t.flags = (i % 2 == 0 && c.se_table.size() > 4096 * 8) ? BS_REF_FLAG_SE_SCALAR : 0u;
      work += (bs_refcodec_serial_work_bytes(c.n, c.ns) + 255) & ~255ull;
      mant_g += (c.nb + per - 1) / per;
      tiles += c.ns * bs_refcodec_serial_tiles(c.n, c.ns);
      streams += c.ns;
    }
    Buf d_tasks(nt * sizeof(bs_ref_task)), d_work(work, true);
    memcpy(d_tasks.p, tasks.data(), nt * sizeof(bs_ref_task));
    int32_t status = 0;
    const int rc = bs_refcodec_decode_serial_batch((const bs_ref_task*)d_tasks.p, (uint32_t)nt, 8u * C, mant_g, tiles,
                                                   streams, d_work.p, work, &status, nullptr);
    for (size_t i = 0; i < nt; ++i) {
      const CleanRef& c = clean_ref[i];
      if (rc == BS_OK && status == 0 && memcmp(outs[i], c.want.data(), c.n * 2) == 0) {
        ++ref_batch_ok;
      } else {
        ++clean_bad;
        fprintf(stderr, "reference batch with gaps, task %zu (n %llu): rc %d status 0x%x\n", i,
                (unsigned long long)c.n, rc, status);
      }
    }
    for (Buf* b : keep) delete b;
  }
  printf("batched tasks ok %llu failed %llu, pointers with bit 31 set %llu, empty task flagged %llu, "
         "reference batch with gaps ok %llu\n",
         (unsigned long long)batch_ok, (unsigned long long)batch_bad, (unsigned long long)high_bit,
         (unsigned long long)empty_flagged, (unsigned long long)ref_batch_ok);
  printf("cases %u clean ok %llu clean failed %llu corrupted: refused %llu flagged %llu decoded %llu "
         "scalar-table mismatches %llu\n", n_cases,
         (unsigned long long)clean_ok, (unsigned long long)clean_bad, (unsigned long long)refused_host,
         (unsigned long long)flagged, (unsigned long long)decoded, (unsigned long long)scalar_mismatch);
  return clean_bad == 0 && scalar_mismatch == 0 ? 0 : 1;
}
