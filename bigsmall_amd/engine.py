"""The decode engine: container entries -> device tensors, on one GPU.

Every caller of the drop-in API (decoder.load/decompress, StreamingLoader,
BigSmallStreamingModel) goes through `GroupDecoder`. A *group* is a set of
container entries decoded together, normally one transformer layer
(bigsmall/streaming.py:218-227 decodes a layer tensor by tensor; here it is
one launch per codec family):

  1. the group's compressed bytes (one contiguous span of the data section)
     are read into a pinned buffer in parallel 16 MB pieces and copied
     host -> device on a copy stream piece by piece as the reads complete;
     the pinned buffers rotate, so the read of group g+1 overlaps the copy of g;
  2. the decode stream waits for that copy only, then launches
       - one batched BSCK launch (bs_chunk_decode_batch) for every
         bf16_chunked_v1 / fp8_chunked_v1 entry of the group,
       - one bs_refcodec_decode_serial_batch launch for the group's
         reference-format entries (bf16_parallel_v1, bf16_se_tans,
         bf16_se_single_kernel) of 65,536 elements or more, so all their
         chains run side by side, and bs_refcodec_decode per smaller one,
       - one bs_zstd_decode launch for the group's zstd frames (`zstd`,
         `zstd_xor_delta` and the index streams of `special` lowcard
         entries), then bs_lut_expand per lowcard entry,
       - device-to-device copies for `raw` entries,
     writing straight into freshly allocated output tensors;
  3. tied entries become copies of their master after it is decoded.
So decoding group g overlaps the host->device copy of group g+1.

Codecs whose bitstream is defined by libraries this engine does not carry
(constriction's bf16_se_rans / bf16_se_ac / fp8_cat_ac / ..., blosc2's
`special` wpe_delta) raise BigSmallVersionError naming the codec.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

from .codecs import _refstreams
from .codecs import bf16_chunked
from .codecs import zstd_gpu
from .container import tensor_numel
from .device import ChunkBatch, ChunkJob, StatusWord, require_gpu
from .exceptions import BigSmallVersionError
from .formats import torch_dtype

BSCK_CODECS = {bf16_chunked.CODEC_BF16: 2, bf16_chunked.CODEC_FP8: 1, bf16_chunked.CODEC_BF16_TANS: 2,
               bf16_chunked.CODEC_FP8_TANS: 1}
REF_CODECS = set(_refstreams.PARSERS)
UNSUPPORTED = {
    "bf16_se_rans": "constriction ANS (Rust library, not available to this engine)",
    "bf16_se_ac": "constriction range coder (Rust library, not available to this engine)",
    "fp8_cat_ac": "constriction range coder", "fp4_cat_ac": "constriction range coder",
    "fp16_se_ac": "constriction range coder", "fp32_se_ac": "constriction range coder",
    "bf16_sparsity_v1": "constriction-coded populations", "fp2_residual_v1": "constriction-coded residual",
    "special": "blosc2 (wpe_delta)",
}
ZSTD_CODECS = {"zstd", "zstd_xor_delta"}


def entry_numel(t: dict) -> int:
    """Element count the way the reference's _decode_blob computes it (decoder.py:53)."""
    return tensor_numel(t) if t["shape"] else 1


def is_lowcard(t: dict) -> bool:
    return t["codec"] == "special" and (t.get("extra") or {}).get("special_kind") == "lowcard"


def tied_copy(src, t: dict):
    """A tied_ref follower: its master's bytes under the follower's own dtype
    and shape. The reference hands the master's raw bytes to the follower's
    _raw_to_numpy (bigsmall/decoder.py:138-155, bigsmall/streaming.py:163-190),
    and its encoder ties entries by (item size, shape, md5) whatever their
    dtypes (bigsmall/tensor_analysis.py:97-110), so F32 and I32 zeros, or BF16
    and F16 words, can share one blob."""
    import torch
    dt = torch_dtype(t["dtype"])
    shape = [int(s) for s in t["shape"]]
    if src.dtype == dt and list(src.shape) == shape:
        return src.clone()
    raw = src.contiguous().view(-1)
    raw = raw.view(torch.uint8) if raw.numel() else raw.to(torch.uint8)
    need = tensor_numel(t) * torch.empty((), dtype=dt).element_size()
    if raw.numel() != need:
        raise ValueError(f"tied_ref {t['name']!r}: master holds {raw.numel()} bytes, "
                         f"{t['dtype']} {shape} needs {need}")
    return raw.clone().view(dt).reshape(shape)


def check_supported(t: dict) -> None:
    codec = t["codec"]
    if codec in ("raw", "tied_ref") or codec in BSCK_CODECS or codec in REF_CODECS or codec in ZSTD_CODECS:
        return
    if is_lowcard(t):
        return
    from . import __version__
    detail = f"file references codec {codec!r}"
    if codec in UNSUPPORTED:
        detail += f", whose bitstream is defined by {UNSUPPORTED[codec]}; the MI355X engine decodes " \
                  f"bf16_chunked_v1, fp8_chunked_v1, bf16_chunked_tans_v1, fp8_chunked_tans_v1, bf16_parallel_v1, " \
                  f"bf16_se_tans, bf16_se_single_kernel, " \
                  f"zstd, zstd_xor_delta, special (lowcard) and raw"
    raise BigSmallVersionError(required="newer-than-installed", installed=__version__, detail=detail)


@dataclass
class GroupResult:
    """Outputs of one decoded group. `tensors` hold valid data once the decode
    stream has passed `done` (call `wait()` to synchronise and check)."""
    tensors: dict
    status: StatusWord
    done: object = None                   # torch.cuda.Event on the decode stream
    keep: list = field(default_factory=list)

    def wait(self, what: str = "decode") -> dict:
        """Synchronise with the decode, check its status word, and hand the
        tensors to the caller's current stream: record_stream keeps the
        allocator from reusing their memory for later decodes (on the decode
        stream) while work the caller queues on its own stream still reads them."""
        import torch
        if self.done is not None:
            self.done.synchronize()
        else:
            torch.cuda.synchronize()
        self.status.check(what)
        self.keep.clear()
        for t in self.tensors.values():
            if t.is_cuda and t.numel():
                t.record_stream(torch.cuda.current_stream(t.device))
        return self.tensors


class GroupDecoder:
    """Decodes groups of container entries into device tensors.

    stream: the decode stream (default: torch's current stream; "private" for a
        new stream of its own, whose outputs the caller then orders with
        `GroupResult.wait`, which also records them on the caller's stream).
    copy_stream: where host->device copies run (default: a new stream).
    Pinned staging buffers are allocated lazily and reused (n_pinned of them).
    pipeline: consecutive groups alternate between the decode stream and a
        second stream of the decoder's own, so that a group's decode starts
        while the previous one's last workgroups finish (its prologue over the
        other's tail: 137 against 144 us per 8B-shaped layer). A group's
        inputs reach its stream through the copy's event; results are ordered
        for the caller by `GroupResult.wait`, which every caller uses.
    """

    def __init__(self, device=None, stream=None, copy_stream=None, n_pinned: int = 2, pipeline: bool = True):
        import torch
        self.device = require_gpu(device)
        if isinstance(stream, str):
            if stream != "private":
                raise ValueError(f"GroupDecoder: stream must be a torch stream, None or 'private', got {stream!r}")
            stream = torch.cuda.Stream(self.device)
        self.stream = stream if stream is not None else torch.cuda.current_stream(self.device)
        self.copy_stream = copy_stream if copy_stream is not None else torch.cuda.Stream(self.device)
        self._decode_streams = [self.stream, torch.cuda.Stream(self.device)] if pipeline else [self.stream]
        self._turn = 0
        self._pinned: list = [None] * max(1, n_pinned)
        self._pinned_busy: list = [None] * len(self._pinned)
        self._next = 0

    # -- staging ---------------------------------------------------------------
    def _pinned_buffer(self, nbytes: int):
        import torch
        i = self._next
        self._next = (self._next + 1) % len(self._pinned)
        ev = self._pinned_busy[i]
        if ev is not None:
            ev.synchronize()              # the copy that last read this buffer has finished
        buf = self._pinned[i]
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, pin_memory=True)
            self._pinned[i] = buf
        return i, buf

    def upload(self, read_span, offset: int, nbytes: int):
        """Copy data-section bytes [offset, offset + nbytes) to a new device
        buffer through a pinned staging buffer; returns (device tensor, the
        pinned bytes as numpy, event recorded after the copy). The copy of
        each piece the reader reports (`read_span(..., on_piece=...)`, in
        order) is queued on the copy stream as soon as that piece is read, so
        the disk/page-cache read and the PCIe transfer of one span overlap."""
        import torch
        i, buf = self._pinned_buffer(nbytes)
        view = buf[:nbytes]
        dev = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)
        dev.record_stream(self.copy_stream)     # freed early (a read error), it outlives queued copies

        def on_piece(p0: int, p1: int) -> None:
            with torch.cuda.stream(self.copy_stream):
                dev[p0:p1].copy_(view[p0:p1], non_blocking=True)

        if nbytes:
            if getattr(read_span, "pieces", False):
                read_span(offset, view.numpy(), on_piece=on_piece)
            else:
                read_span(offset, view.numpy())
                on_piece(0, nbytes)
        with torch.cuda.stream(self.copy_stream):
            ev = torch.cuda.Event()
            ev.record(self.copy_stream)
        self._pinned_busy[i] = ev
        return dev, view.numpy(), ev

    # -- decoding --------------------------------------------------------------
    def decode_group(self, entries: list[dict], read_span, span_start: int, span_len: int,
                     resolve_tied=None, dtype=None, xor_base: Optional[dict] = None) -> GroupResult:
        """Decode `entries` (container tensor dicts). Their blobs lie in the data
        section range [span_start, span_start + span_len); `read_span(offset,
        np_out)` fills np_out with that many bytes of the data section starting
        at offset. `resolve_tied(name)` returns the decoded master tensor for a
        tied entry whose master is outside the group. `xor_base` maps names of
        zstd_xor_delta entries to their base tensors on this device; such an
        entry decodes to base XOR delta (without a base: to the delta bytes,
        as bigsmall/decoder.py:88-90 returns them)."""
        import torch
        for t in entries:
            check_supported(t)
        d_span, host, copied = self.upload(read_span, span_start, span_len)
        stream = self._decode_streams[self._turn]
        self._turn = (self._turn + 1) % len(self._decode_streams)
        with torch.cuda.stream(stream):            # allocations and launches on this group's decode stream
            status, out, keep = self._launch_group(entries, host, d_span, copied, span_start, span_len,
                                                   resolve_tied, dtype, xor_base or {}, stream)
            done = torch.cuda.Event()
            done.record(stream)
        return GroupResult(out, status, done, keep)

    def _launch_group(self, entries, host, d_span, copied, span_start, span_len, resolve_tied, dtype, xor_base,
                      stream):
        import torch
        status = StatusWord(self.device)
        out: dict = {}
        keep = [d_span]
        jobs = []
        refs = []
        serial_refs = []
        raws = []
        zst = zstd_gpu.ZstdLaunch(self.device)
        base = d_span.data_ptr()
        for t in entries:
            if t["codec"] == "tied_ref":
                continue
            shape = [int(s) for s in t["shape"]]
            tdt = torch_dtype(t["dtype"])
            o = torch.empty(shape, dtype=tdt, device=self.device)
            out[t["name"]] = o
            off, nb = int(t["offset"]) - span_start, int(t["compressed_bytes"])
            if not 0 <= off <= off + nb <= span_len:
                raise ValueError(f"{t['name']}: blob [{t['offset']}, +{nb}) outside its group's span")
            n = entry_numel(t)
            codec = t["codec"]
            if codec == "raw":
                if nb != o.numel() * o.element_size():
                    raise ValueError(f"{t['name']}: raw blob has {nb} bytes, tensor needs "
                                     f"{o.numel() * o.element_size()}")
                raws.append((o, off, nb))
            elif codec in BSCK_CODECS:
                eb = BSCK_CODECS[codec]
                if o.element_size() != eb:
                    raise ValueError(f"{t['name']}: {codec} decodes {eb}-byte elements, dtype is {t['dtype']}")
                if n == 0 or nb == 0:
                    continue
                inf = bf16_chunked.info(bytes(host[off:off + 32]))
                if inf.n != n or inf.elem_bytes != eb:
                    raise ValueError(f"{t['name']}: {codec} weight count mismatch ({inf.n} vs {n})")
                ptr = base + off
                if ptr % 16:
                    # BSCK needs 16-byte aligned blobs: realign on the decode stream (below)
                    a = torch.empty(nb + 16, dtype=torch.uint8, device=self.device)
                    keep.append(a)
                    jobs.append((ChunkJob(a.data_ptr(), nb, o.data_ptr(), n, inf.n_chunks, inf.plane_mode), (off, nb, a)))
                else:
                    jobs.append((ChunkJob(ptr, nb, o.data_ptr(), n, inf.n_chunks, inf.plane_mode), None))
            elif codec in REF_CODECS:
                if o.element_size() != 2:
                    raise ValueError(f"{t['name']}: {codec} decodes bf16, dtype is {t['dtype']}")
                if n == 0 or nb == 0:
                    continue
                plan = _refstreams.PARSERS[codec](bytes(host[off:off + nb]), n)
                if _refstreams.serial_ok(plan):
                    serial_refs.append((plan, base + off, o.data_ptr()))
                else:
                    refs.append((_refstreams.RefLaunch(plan, base + off, self.device), o))
            elif codec in ZSTD_CODECS:
                if nb == 0:
                    raise ValueError(f"{t['name']}: empty {codec} blob")
                nbytes = o.numel() * o.element_size()
                xb = xor_base.get(t["name"]) if codec == "zstd_xor_delta" else None
                if xb is not None:
                    if not xb.is_contiguous() or xb.numel() * xb.element_size() != nbytes or xb.device != o.device:
                        raise ValueError(f"Delta size mismatch for {t['name']}")
                    keep.append(xb)
                zst.add_frame(base + off, nb, o.data_ptr(), nbytes, xb.data_ptr() if xb is not None else 0)
            else:                                        # special/lowcard (check_supported)
                zst.add_lowcard(base + off, host[off:off + nb], o.data_ptr(), o.numel(), o.element_size())
        stream.wait_event(copied)
        d_span.record_stream(stream)
        for o, off, nb in raws:
            o.view(-1).view(torch.uint8).copy_(d_span[off:off + nb])
        if jobs:
            for job, realign in jobs:
                if realign is not None:
                    off, nb, a = realign
                    a[:nb].copy_(d_span[off:off + nb])
            batch = ChunkBatch([j for j, _ in jobs], self.device)
            keep.append(batch)
            batch.launch(status, stream)
        if serial_refs:
            # every large reference-format tensor of the group in one batched
            # wave-serial launch: their chains run side by side
            rb = _refstreams.RefBatch(serial_refs, self.device)
            keep.append(rb)
            rb.launch(status.ptr, int(stream.cuda_stream))
        for launch, o in refs:
            keep.append(launch)
            launch.launch(o.data_ptr(), status.ptr, int(stream.cuda_stream))
        if zst.tasks or zst.expands:
            zst.launch(status, stream)
            keep.append(zst.keep)
        for t in entries:
            if t["codec"] != "tied_ref":
                continue
            master = (t.get("extra") or {}).get("tied_to")
            src = out.get(master)
            if src is None and resolve_tied is not None:
                src = resolve_tied(master)
            if src is None:
                raise KeyError(f"tied_ref master {master!r} of {t['name']!r} not found")
            out[t["name"]] = tied_copy(src, t)
        if dtype is not None:
            for k, v in out.items():
                if v.is_floating_point() and v.dtype != dtype:
                    out[k] = v.to(dtype)
        return status, out, keep


READ_PIECE = 16 << 20          # bytes per parallel read of a span


def file_span_reader(path, threads: Optional[int] = None):
    """read_span(offset, np_out) over the data section of a container file.
    Spans above READ_PIECE are read in pieces by `threads` threads at once
    (pread releases the GIL), so filling a pinned staging buffer from the page
    cache runs at memory speed rather than one thread's copy rate."""
    from .container import read_header
    _, data_offset = read_header(path)
    fd = os.open(str(path), os.O_RDONLY)
    # 4 readers: more measured no faster on the GPU host and slower at 16 (they compete with the
    # caller's own threads for the host's cores)
    n_threads = threads if threads is not None else max(1, min(4, os.cpu_count() or 1))
    pool = ThreadPoolExecutor(n_threads, thread_name_prefix="bs-read") if n_threads > 1 else None

    def read_range(mv: memoryview, offset: int) -> None:
        got = 0
        while got < len(mv):
            k = os.preadv(fd, [mv[got:]], data_offset + offset + got)
            if k <= 0:
                raise ValueError(f"{path}: data section truncated at {offset + got}")
            got += k

    def read_span(offset: int, dst: np.ndarray, on_piece=None) -> None:
        """Fill dst; on_piece(p0, p1), if given, is called in order from this
        thread as each piece [p0, p1) of dst is complete."""
        mv = memoryview(dst).cast("B")
        n = len(mv)
        if pool is None or n <= READ_PIECE:
            read_range(mv, offset)
            if on_piece is not None and n:
                on_piece(0, n)
            return
        starts = range(0, n, READ_PIECE)
        futs = [pool.submit(read_range, mv[p:p + READ_PIECE], offset + p) for p in starts]
        try:
            for p, f in zip(starts, futs):
                f.result()
                if on_piece is not None:
                    on_piece(p, min(n, p + READ_PIECE))
        finally:
            for f in futs:          # no read may still write into dst after an error
                f.cancel()
            for f in futs:
                if not f.cancelled():
                    f.exception()

    def close() -> None:
        if pool is not None:
            pool.shutdown(wait=True)
        os.close(fd)

    read_span.close = close
    read_span.pieces = True
    return read_span


def group_span(entries: list[dict]) -> tuple[int, int]:
    """[start, end) of the data section holding the entries' blobs."""
    ents = [t for t in entries if t["codec"] != "tied_ref" and int(t["compressed_bytes"]) > 0]
    if not ents:
        return 0, 0
    lo = min(int(t["offset"]) for t in ents)
    hi = max(int(t["offset"]) + int(t["compressed_bytes"]) for t in ents)
    return lo, hi


__all__ = ["GroupDecoder", "GroupResult", "check_supported", "entry_numel", "file_span_reader", "group_span",
           "BSCK_CODECS", "REF_CODECS", "UNSUPPORTED"]
