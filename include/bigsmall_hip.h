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
 * negative BS_ERR_* codes. No entry point keeps global mutable state; calls on
 * different streams with disjoint buffers may run concurrently.
 *
 * Reference interfaces replaced (paths relative to the reference checkout):
 *   bs_chunk_*   — new GPU-native codec registered through the reference's
 *                  plugin API `codec_registry.register_codec(name, enc, dec)`
 *                  (bigsmall/codec_registry.py:45-47) and dispatched from the
 *                  decoder's `_decode_blob` chain (bigsmall/decoder.py:49-97).
 *   bs_par1_*    — `kernels.decode_bf16_parallel(blob, extras, n_weights)`
 *                  (bigsmall/kernels/__init__.py:89-111) and the CPU decode it
 *                  must match, `bf16_parallel.decode` (bigsmall/codecs/bf16_parallel.py:262-352).
 *   bs_tans_*    — `bf16_tans.decode` (bigsmall/codecs/bf16_tans.py:121-167).
 *   bs_sk_*      — `single_kernel.decode` (bigsmall/codecs/single_kernel.py:603-613).
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
/* BSCK: GPU-native chunked rANS format ("bf16_chunked_v1" / "fp8_chunked_v1").
 * Registered through codec_registry.register_codec (bigsmall/codec_registry.py:45-47). */

typedef struct {
    uint64_t n;          /* elements */
    uint32_t n_chunks;
    uint32_t steps;      /* rANS steps per lane per full chunk */
    uint32_t lanes;      /* interleaved rANS states per chunk (64 or 128) */
    uint32_t n_syms;
    uint32_t elem_bytes; /* 2 = bf16 words, 1 = bytes (fp8) */
    uint32_t plane_mode; /* 0 none, 1 dense, 2 compact */
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
 * launch; `max_plane_mode` is the largest plane_mode among the tasks (mode 2
 * launches reserve extra LDS for the compact-plane rings). Replaces the per-tensor `_decode_blob` loop of decoder.decompress
 * (bigsmall/decoder.py:128-136) and StreamingLoader.load_layer
 * (bigsmall/streaming.py:218-227). */
int bs_chunk_decode_batch(const bs_chunk_task *d_tasks, uint32_t n_tasks, uint32_t total_groups,
                          uint32_t max_plane_mode, int32_t *d_status, void *stream);

/* Host encoder for BSCK. `flags`: BS_CHUNK_MODE_AUTO or a forced plane mode.
 * Replaces the encode half of the codec plugin pair (bigsmall/codec_registry.py:39-47). */
#define BS_CHUNK_MODE_AUTO (-1)
int bs_chunk_encode_bound(uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, uint64_t *bound);
int bs_chunk_encode(const void *h_src, uint64_t n, uint32_t elem_bytes, uint32_t lanes, uint32_t steps, int32_t mode,
                    uint8_t *h_dst, uint64_t cap, uint64_t *out_len, int n_threads);

#ifdef __cplusplus
}
#endif

#endif /* BIGSMALL_HIP_H */
