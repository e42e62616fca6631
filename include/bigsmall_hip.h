/*
 * bigsmall_hip.h — C ABI of the MI355X BigSmall decode engine
 * (libbigsmall_hip.so, built from bigsmall_amd/csrc/).
 *
 * Plain pointers and sizes only. "d_" pointers are device (HBM) pointers,
 * "h_" pointers are host pointers. `stream` is a hipStream_t passed as void*
 * (NULL = the legacy default stream). Every decode entry point is
 * asynchronous on `stream`; integrity failures found on the device are OR-ed
 * into the caller-provided device word `d_status` (BS_DEV_* bits), which the
 * caller reads after synchronising. Host-side failures are returned as
 * negative BS_ERR_* codes. No entry point keeps global mutable state, except
 * bs_zstd_decode_static (a static device work area and an ordering event per
 * GPU, below); calls on different streams with disjoint buffers may run
 * concurrently.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   bs_chunk_*   — new GPU-native codec registered through the reference's
 *                  plugin API `codec_registry.register_codec(name, enc, dec)`
 *                  (bigsmall/codec_registry.py:45-47) and dispatched from the
 *                  decoder's `_decode_blob` chain (bigsmall/decoder.py:49-97).
 *   bs_chunk_encode_gpu — the host encode of the KV-cache entry codec
 *                  (bigsmall/codecs/kv_cache.py:41-83) for device-resident tensors.
 *   bs_refcodec_decode — `kernels.decode_bf16_parallel(blob, extras, n_weights)`
 *                  (bigsmall/kernels/__init__.py:89-111) and the CPU decoders it
 *                  must match: `bf16_parallel.decode` (bigsmall/codecs/bf16_parallel.py:262-352),
 *                  `bf16_tans.decode` (bigsmall/codecs/bf16_tans.py:121-167),
 *                  `single_kernel.decode` (bigsmall/codecs/single_kernel.py:603-613).
 */
#ifndef BIGSMALL_HIP_H
#define BIGSMALL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* host return codes */
#define BS_OK 0
#define BS_ERR_ARG (-1)     /* bad argument (null pointer, misalignment, size) */
#define BS_ERR_FORMAT (-2)  /* malformed blob header */
#define BS_ERR_CAP (-3)     /* output capacity too small */
#define BS_ERR_HIP (-4)     /* HIP runtime error (launch failure) */
#define BS_ERR_COUNT (-5)   /* element count does not match the blob */

/* device status bits (OR-ed into *d_status by the kernels) */
#define BS_DEV_ERR_HEADER 0x1  /* bad magic / version / field out of range */
#define BS_DEV_ERR_COUNT 0x2   /* blob element count != requested count */
#define BS_DEV_ERR_BOUNDS 0x4  /* a section lies outside the blob */
#define BS_DEV_ERR_STREAM 0x8  /* a stream did not end in the encoder's start state */

/* Library version: major*10000 + minor*100 + patch. No reference counterpart. */
int bs_version(void);

/* ------------------------------------------------------------------------ */
/* BSCK: GPU-native chunked entropy-coded format, rANS ("bf16_chunked_v1" /
 * "fp8_chunked_v1") or tANS ("bf16_chunked_tans_v1" / "fp8_chunked_tans_v1").
 * Registered through codec_registry.register_codec (bigsmall/codec_registry.py:45-47). */

typedef struct {
    uint64_t n;          /* elements */
    uint32_t n_chunks;
    uint32_t steps;      /* steps per lane per full chunk */
    uint32_t lanes;      /* interleaved states per chunk (64, 128 or 256) */
    uint32_t n_syms;
    uint32_t elem_bytes; /* 2 = bf16 words, 1 = bytes (fp8) */
    uint32_t plane_mode; /* 0 none, 1 dense, 2 compact, 3 fp8 exponent pairs + dense plane */
    uint32_t coder;      /* 0 rANS; tANS: 1 (u32 state array), 2 (12-bit states at the stream head) */
} bs_chunk_info;

/* One tensor of a batched launch (device-resident array of these). */
typedef struct {
    const uint8_t *blob; /* device, 16-byte aligned */
    uint64_t blob_bytes;
    void *out;           /* device, n * elem_bytes bytes */
    uint64_t n;
    uint32_t wg_begin;   /* first workgroup of this tensor within the grid */
    uint32_t n_chunks;
} bs_chunk_task;

/* Parse a BSCK header from host bytes (the first 32 bytes suffice).
 * Replaces the header read that bf16_parallel._unpack_header does on the host
 * (bigsmall/codecs/bf16_parallel.py:138-183) for the GPU-native format. */
int bs_chunk_inspect(const uint8_t *h_blob, uint64_t len, bs_chunk_info *info);

/* Number of chunks one workgroup decodes (tasks[i].wg_begin spacing is
 * ceil(n_chunks / bs_chunk_chunks_per_group())). */
int bs_chunk_chunks_per_group(void);

/* Decode one BSCK blob into d_out (16-byte aligned). `plane_mode` is the header's (from
 * bs_chunk_inspect). Device counterpart of the codec plugin's
 * decode(blob, extras, n_weights) (bigsmall/codec_registry.py:39-42). */
int bs_chunk_decode(const uint8_t *d_blob, uint64_t blob_bytes, void *d_out, uint64_t n,
                    uint32_t n_chunks, uint32_t plane_mode, int32_t *d_status, void *stream);

/* Decode many BSCK blobs (a transformer layer, a batch of KV blocks) in one
 * launch, rANS and tANS blobs alike; `max_plane_mode` is the largest
 * plane_mode among the tasks (a launch whose tasks are all of modes 0 and 1
 * uses a kernel built without the compact-plane path; both use the same LDS
 * and occupancy). Tasks are in ascending wg_begin order,
 * task 0 at 0, each starting where the previous one's workgroups end; every
 * blob and output is 16-byte aligned, and total_groups is the last task's end
 * (a workgroup serves the last task whose wg_begin is at or before it, so
 * a table out of order decodes some tensors into the wrong place but never
 * reads or writes outside the tasks' buffers). Replaces the per-tensor `_decode_blob`
 * loop of decoder.decompress
 * (bigsmall/decoder.py:128-136) and StreamingLoader.load_layer
 * (bigsmall/streaming.py:218-227). */
int bs_chunk_decode_batch(const bs_chunk_task *d_tasks, uint32_t n_tasks, uint32_t total_groups,
                          uint32_t max_plane_mode, int32_t *d_status, void *stream);

/* Host encoder for BSCK. `mode`: BS_CHUNK_MODE_AUTO or a forced plane mode
 * (0-2 for bf16; 0 or 3 for bytes, 3 needing an even n). `coder`: 0 rANS,
 * 1 or 2 tANS (2, the smaller, keeps a chunk's 12-bit initial states at the
 * head of its bit stream; 1 stores them as u32 words, the layout of earlier
 * blobs, which still decode). bs_chunk_encode is bs_chunk_encode_ex with coder 0, and
 * bs_chunk_encode_bound its capacity (bs_chunk_encode_bound_ex for either
 * coder). Replaces the encode half of the codec plugin pair
 * (bigsmall/codec_registry.py:39-47). */
#define BS_CHUNK_MODE_AUTO (-1)
int bs_chunk_encode_bound(uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, uint64_t *bound);
int bs_chunk_encode_bound_ex(uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, int32_t coder,
                             uint64_t *bound);
int bs_chunk_encode(const void *h_src, uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, int32_t mode,
                    uint8_t *h_dst, uint64_t cap, uint64_t *out_len, int n_threads);
int bs_chunk_encode_ex(const void *h_src, uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps,
                       int32_t mode, int32_t coder, uint8_t *h_dst, uint64_t cap, uint64_t *out_len, int n_threads);

/* GPU encoder for BSCK, for tensors already in HBM (bf16, dense plane mode,
 * 128 states per chunk). A batch of tasks sorted by chunk_begin; task i owns
 * global chunks [chunk_begin, chunk_begin + n_chunks), chunks numbered
 * consecutively from 0 over the batch (total_chunks in all). Blobs are
 * byte-identical to bs_chunk_encode(..., elem_bytes 2, lanes 128, mode 1).
 * Replaces the host encode of the KV-cache entry codec
 * (bigsmall/codecs/kv_cache.py:41-83, which copies the tensor to the host and
 * encodes there) for device-resident K/V blocks. */
typedef struct {
    const void *src;      /* n bf16 words (device, 4-byte aligned), n >= 1, n < 2^32 */
    uint64_t n;
    uint8_t *dst;         /* blob output (device, 16-byte aligned) */
    uint64_t cap;         /* dst capacity, e.g. bs_chunk_encode_bound(n, 2, 128, steps) */
    uint32_t chunk_begin;
    uint32_t n_chunks;    /* ceil(n / (128 * steps)) */
    /* Where the words lie: seg_len 0, contiguous (word e at src + e); else in
     * segments of seg_len words (a multiple of 512) whose starts are
     * seg_stride words apart (seg_stride >= seg_len, a multiple of 8): word e
     * at src + (e / seg_len) * seg_stride + e % seg_len, every word below
     * 2^32 from src. A block of tokens of a [heads, tokens, dim] KV tensor is
     * such a task, read in place. */
    uint64_t seg_len;
    uint64_t seg_stride;
} bs_encode_task;

/* Device scratch bytes bs_chunk_encode_gpu needs. */
uint64_t bs_chunk_encode_gpu_work_bytes(uint32_t n_tasks, uint64_t total_chunks, uint32_t steps);

/* Encode every task on `stream`. d_out_len[i] receives blob i's length (0 if
 * the task failed: BS_DEV_ERR_HEADER for inconsistent task fields,
 * BS_DEV_ERR_BOUNDS for a blob larger than its capacity, OR-ed into
 * *d_status). d_work: 256-byte aligned scratch of the size above. */
int bs_chunk_encode_gpu(const bs_encode_task *d_tasks, uint32_t n_tasks, uint32_t total_chunks, uint32_t steps,
                        void *d_work, uint64_t work_bytes, uint64_t *d_out_len, int32_t *d_status, void *stream);

/* Copy n_spans device byte ranges on `stream`, e.g. to pack the encoder's
 * blobs (written at their worst-case slots) back to back. Every src, dst and
 * len must be a multiple of 16 (a span that is not sets BS_DEV_ERR_HEADER in
 * *d_status and is skipped); spans must not overlap one another's dst.
 * max_len (>= every len) sizes the launch. Replaces the host byte
 * concatenation that frames KV entries (bigsmall/codecs/kv_cache.py:74-83)
 * for blobs that stay in HBM. */
typedef struct {
    const uint8_t *src;
    uint8_t *dst;
    uint64_t len;
} bs_span;
int bs_copy_spans(const bs_span *d_spans, uint32_t n_spans, uint64_t max_len, int32_t *d_status, void *stream);

/* ------------------------------------------------------------------------ */
/* The reference's rANS-family bf16 formats, decoded on the GPU:
 *   bf16_parallel_v1      (bigsmall/codecs/bf16_parallel.py:262-352; the entry
 *                          kernels.decode_bf16_parallel, bigsmall/kernels/__init__.py:89-111)
 *   bf16_se_tans          (bigsmall/codecs/bf16_tans.py:121-167)
 *   bf16_se_single_kernel (bigsmall/codecs/single_kernel.py:603-613)
 * The host parses the blob header (bigsmall_amd/codecs/_refstreams.py) into
 * stream descriptors and decode tables; these two kernels do all symbol work. */

/* One rANS stream: initial state x0, then n_words little-endian u16 words at
 * `words` (device, any alignment). If bit 16 of `tail` is set, one more word
 * with value (tail & 0xFFFF) follows (an odd trailing byte in the reference's
 * framing). */
typedef struct {
    const uint8_t *words;
    uint32_t x0;
    uint32_t n_words;
    uint32_t tail;
    uint32_t n;          /* symbols */
    uint64_t first;      /* element index of the first symbol */
    uint32_t stride;     /* element index step between symbols */
    uint32_t reserved;
} bs_se_stream;

typedef struct {
    const uint8_t *words;
    uint32_t x0;
    uint32_t n_words;
    uint32_t tail;
    uint32_t n;          /* mantissas in the bucket */
    uint64_t perm_begin; /* index in perm of the bucket's first element */
    uint32_t table;      /* mantissa table index */
    uint32_t reserved;
} bs_mant_bucket;

/* Decode one tensor of a reference rANS-family format into d_out (n_out bf16
 * words). d_se_table: 4096 x {f | (slot-cf) << 13, symbol} u32 pairs.
 * d_bstart: n_streams x 257 u32, the perm index where the bucket of exponent e
 * of each stream starts (entry 256 = the stream's end). d_mant_tables:
 * n_tables x 1024 u32 {f | (slot-cf) << 11 | symbol << 21}. d_perm: n_out u32
 * of scratch. Asynchronous on `stream`; device integrity failures are OR-ed
 * into *d_status. Replaces the CPU decode loops of bf16_parallel.decode,
 * bf16_tans.decode and single_kernel._decode_full_kernel (paths above) and the
 * SE-only Triton kernel (bigsmall/kernels/ac_triton.py:47-102). */
int bs_refcodec_decode(const bs_se_stream *d_streams, uint32_t n_streams, const uint32_t *d_se_table,
                       const uint32_t *d_bstart, const bs_mant_bucket *d_buckets, uint32_t n_buckets,
                       const uint32_t *d_mant_tables, uint32_t n_tables, uint16_t *d_out, uint64_t n_out,
                       uint32_t *d_perm, int32_t *d_status, void *stream);

/* Workspace bytes bs_refcodec_decode_serial needs for n_out elements in n_streams SE streams. */
uint64_t bs_refcodec_serial_work_bytes(uint64_t n_out, uint32_t n_streams);

/* The same formats and descriptors as bs_refcodec_decode, decoded with one
 * wavefront per chain: every SE stream (N for bf16_parallel_v1,
 * bigsmall/codecs/bf16_parallel.py:262-352; one for bf16_se_tans,
 * bigsmall/codecs/bf16_tans.py:121-167, and bf16_se_single_kernel,
 * bigsmall/codecs/single_kernel.py:431-580) and every mantissa bucket, SE and
 * mantissa chains at the same time, then a parallel stable counting sort by
 * exponent within each stream places the mantissas. Streams must each hold at
 * most ceil(n_out / n_streams) symbols. d_work: bs_refcodec_serial_work_bytes
 * bytes of device scratch, 256-byte aligned. Replaces the serial decode loops
 * of rans.decode_stream (bigsmall/codecs/rans.py:165-207),
 * numba_rans._decode_kernel (bigsmall/codecs/numba_rans.py:168-192) and
 * single_kernel._decode_full_kernel. n_out < 2^32. Asynchronous on `stream`;
 * integrity failures OR-ed into *d_status. */
int bs_refcodec_decode_serial(const bs_se_stream *d_streams, uint32_t n_streams, const uint32_t *d_se_table,
                              const uint32_t *d_bstart, const bs_mant_bucket *d_buckets, uint32_t n_buckets,
                              const uint32_t *d_mant_tables, uint32_t n_tables, uint16_t *d_out, uint64_t n_out,
                              void *d_work, uint64_t work_bytes, int32_t *d_status, void *stream);

/* Tiles per SE stream of the placement passes of the wave-serial path (the
 * tile grid of a task holds n_streams x this many workgroups). */
uint32_t bs_refcodec_serial_tiles(uint64_t n_out, uint32_t n_streams);

/* One tensor of a batched wave-serial launch: the descriptors, tables and
 * output of bs_refcodec_decode_serial, plus where the task sits in the batch.
 * The chains run in workgroups of bs_refcodec_serial_chains_per_group()
 * wavefronts: first every task's SE groups (ceil(n_streams / per group) each,
 * from se_group_begin), then every task's mantissa-bucket groups
 * (ceil(n_buckets / per group) each, from mant_group_begin, counted from the
 * end of the SE groups), so the longest chains start first. A task's
 * workgroups are consecutive in each grid; across the task array (device
 * memory) every *_begin ascends, and a task's range starts at or after the
 * previous one's end (the workgroups of a gap exit at once). The SE part of
 * the chain grid is dealt to the XCDs in bins: with total_se_groups rounded up
 * to 8C, slot p (which the round-robin dispatch sends to XCD p % 8) decodes SE
 * group (p % 8) * C + p / 8, so XCD j decodes groups [jC, (j+1)C). A caller
 * that places each task's SE groups inside one bin (gaps where needed) keeps
 * the tasks whose tables are read through the scalar cache on XCDs of their
 * own. */
typedef struct {
    const bs_se_stream *streams;     /* n_streams SE stream descriptors */
    const uint32_t *se_table;        /* 4096 x {f | (slot-cf) << 13, symbol} u32 pairs */
    const uint32_t *bstart;          /* n_streams x 257 u32 */
    const bs_mant_bucket *buckets;   /* n_buckets */
    const uint32_t *mant_tables;     /* n_tables x 1024 u32 */
    uint16_t *out;                   /* n_out bf16 words */
    uint64_t n_out;                  /* 1 .. 2^32 - 1 */
    uint64_t work_offset;            /* multiple of 256: the task's bs_refcodec_serial_work_bytes(n_out,
                                        n_streams) bytes of scratch start at d_work + work_offset */
    uint32_t n_streams, n_buckets, n_tables;
    uint32_t se_group_begin;         /* chain grid, SE part: ceil(n_streams / per group) workgroups */
    uint32_t tile_begin;             /* tile grid: n_streams x bs_refcodec_serial_tiles(n_out, n_streams) */
    uint32_t stream_begin;           /* stream grid: n_streams */
    uint32_t mant_group_begin;       /* chain grid, mantissa part: ceil(n_buckets / per group) workgroups */
    uint32_t flags;                  /* BS_REF_FLAG_* */
} bs_ref_task;

/* bs_ref_task.flags. BS_REF_FLAG_SE_SCALAR: se_table continues after its 4096
 * pairs with the table's 4-byte form, 4096 u32 {index | f << 8 | (slot - cf)
 * << 20}, and 256 u32 output words (sign << 15 | exponent << 7 of the SE
 * symbol with that index), which a tensor with at most 256 live SE symbols,
 * none of frequency 4096, has; its SE chains then keep their state in scalar
 * registers and read that table through the scalar cache. BS_REF_FLAG_MANT_SCALAR:
 * the mantissa chains do the same with mant_tables. Either way the decoded
 * words are the same. */
#define BS_REF_FLAG_SE_SCALAR 1u
#define BS_REF_FLAG_MANT_SCALAR 2u

/* Wavefronts (chains) per workgroup of the wave-serial chain grid. */
uint32_t bs_refcodec_serial_chains_per_group(void);

/* Decode every task of d_tasks (a transformer layer's reference-format
 * tensors) with the wave-serial path, all tasks' chains in one launch: the
 * layer takes as long as its longest chain instead of the sum of its tensors'
 * chains. total_* are the grid sizes (the end of the last task's range in each
 * grid). A task whose fields are inconsistent (n_out out of range, no stream,
 * scratch outside d_work) sets BS_DEV_ERR_HEADER and is skipped. Replaces the
 * per-tensor decode loop of decoder.decompress (bigsmall/decoder.py:128-136)
 * and StreamingLoader.load_layer (bigsmall/streaming.py:218-227) for the
 * formats of bs_refcodec_decode_serial. Asynchronous on `stream`. */
int bs_refcodec_decode_serial_batch(const bs_ref_task *d_tasks, uint32_t n_tasks, uint32_t total_se_groups,
                                    uint32_t total_mant_groups, uint32_t total_tiles, uint32_t total_streams,
                                    void *d_work, uint64_t work_bytes, int32_t *d_status, void *stream);

/* Host encoders of the same three formats, for compress() with the
 * reference's gpu_optimised (bf16_parallel_v1) and prefer_speed
 * (bf16_se_single_kernel, bf16_se_tans) choices
 * (bigsmall/codec_registry.py:316-391). `codec`: BS_REF_*; h_src: n bf16
 * words (n < 2^32); n_streams: bf16_parallel_v1's stream count (1..65535,
 * clamped to n like the reference's encoder). The blob is byte-identical to the
 * reference encoder's: bf16_parallel.encode (bigsmall/codecs/bf16_parallel.py:186-259),
 * bf16_tans.encode (bigsmall/codecs/bf16_tans.py:68-118) and
 * single_kernel.encode (bigsmall/codecs/single_kernel.py:193-428, 586-600).
 * *out_len receives its length; a blob longer than cap returns BS_ERR_CAP
 * (cap = bs_refcodec_encode_bound always suffices). An empty tensor is an
 * empty blob. n_threads: host threads for independent streams and buckets. */
#define BS_REF_PARALLEL 0
#define BS_REF_TANS 1
#define BS_REF_SINGLE_KERNEL 2
uint64_t bs_refcodec_encode_bound(int32_t codec, uint64_t n, uint32_t n_streams);
int bs_refcodec_encode(int32_t codec, const uint16_t *h_src, uint64_t n, uint32_t n_streams, uint8_t *h_dst,
                       uint64_t cap, uint64_t *out_len, int n_threads);

/* ------------------------------------------------------------------------ */
/* Zstandard (RFC 8878) frames on the GPU, for the reference's zstd-coded
 * entries: codec "zstd" (bigsmall/codecs/generic.py:15-18, called from
 * bigsmall/decoder.py:80-81), the index stream of "special" lowcard entries
 * (bigsmall/codecs/special.py:67-85) and "zstd_xor_delta" deltas
 * (bigsmall/decoder.py:88-90, 190-198). The reference decodes these with the
 * zstandard package on the host. */
typedef struct {
    const uint8_t *src;   /* one or more zstd (or skippable) frames, back to back (device) */
    uint64_t src_len;
    uint8_t *dst;         /* decoded bytes (device); may be NULL when dst_len is 0 */
    uint64_t dst_len;     /* the exact decoded size */
    const uint8_t *xor_src; /* NULL, or dst_len bytes XOR-ed into the decoded bytes (a delta's base) */
} bs_zstd_task;

/* Device scratch bytes bs_zstd_decode needs (128 KiB per task). */
uint64_t bs_zstd_work_bytes(uint32_t n_tasks);

/* Decode every task on `stream`, one workgroup per task. d_out_len[i]
 * receives task i's decoded byte count (0 if it failed). Failures OR-ed into
 * *d_status: BS_DEV_ERR_HEADER (bad magic, reserved bits, a dictionary
 * frame), BS_DEV_ERR_BOUNDS (truncated input), BS_DEV_ERR_STREAM (invalid
 * table or bitstream, a match before the frame start), BS_DEV_ERR_COUNT (the
 * output is not dst_len bytes, or a frame's is not its recorded content size). Content
 * checksums are skipped, not checked. Dictionaries are not supported. */
int bs_zstd_decode(const bs_zstd_task *d_tasks, uint32_t n_tasks, void *d_work, uint64_t work_bytes,
                   uint64_t *d_out_len, int32_t *d_status, void *stream);

/* bs_zstd_decode without a work buffer, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). No counterpart in the reference. The literal slices
 * live in a static device array of BS_ZSTD_STATIC_MAX_TASKS x 128 KiB (8 MiB)
 * that every GPU the library runs on holds until the process ends; more
 * tasks return BS_ERR_CAP. The call allocates no device memory (the array's
 * address is looked up, and one ordering event created, once per device, on
 * its first call there). All calls on one GPU share the array, and the
 * library orders them: each call's stream waits for the previous call's
 * launch on that GPU (whatever its stream or host thread) before its own
 * launch. Under stream capture that ordering is left to the graph, so
 * launches of two captured graphs that overlap on one GPU race. Otherwise as
 * bs_zstd_decode. */
#define BS_ZSTD_STATIC_MAX_TASKS 64
int bs_zstd_decode_static(const bs_zstd_task *d_tasks, uint32_t n_tasks, uint64_t *d_out_len, int32_t *d_status,
                          void *stream);

/* Lowcard expansion, the unique_bytes[idx] of bigsmall/codecs/special.py:79-82:
 * out[i * item_bytes + b] = lut[idx[i] * item_bytes + b] for i < n, one task
 * per entry (all pointers device). An index >= n_lut sets BS_DEV_ERR_COUNT and
 * leaves its element unwritten; item_bytes outside 1..8 or n_lut > 256 sets
 * BS_DEV_ERR_HEADER. max_n (>= every n) sizes the launch; n_tasks <= 65535. */
typedef struct {
    const uint8_t *idx;
    const uint8_t *lut;
    uint8_t *out;
    uint64_t n;
    uint32_t n_lut;
    uint32_t item_bytes;
} bs_lut_task;
int bs_lut_expand(const bs_lut_task *d_tasks, uint32_t n_tasks, uint64_t max_n, int32_t *d_status, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* BIGSMALL_HIP_H */
