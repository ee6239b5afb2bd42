"""AlphaFold 3 parameter records: the reference's checkpoint format, read straight into HBM.

Format (``xfold/params.py:40-91``), one record after another, little endian:
    header  '<5i': len(scope), len(name), len(dtype), ndim, len(data)
    scope, name, dtype (utf-8 bytes), shape (ndim x '<i'), data (C order)
with dtype one of float32, bfloat16, float16, uint8. A record cut short raises
:class:`RecordError`, as the reference's reader does. A checkpoint may be split over several
files that are read as one byte stream (a record may span two files).

:func:`load_params` reads a checkpoint onto the GPU: a first pass over the headers sizes
one device allocation (every tensor 256-byte aligned inside it), a second pass streams the
payloads through two pinned host buffers whose copies to HBM overlap the file reads. The
result maps ``"scope/name"`` to tensors (views of that allocation), the keys of the
reference's ``get_alphafold3_params``. zstd-compressed checkpoints (``.zst``) need the
``zstandard`` module, which is optional.
"""

from __future__ import annotations

import io
import os
import struct
from pathlib import Path
from typing import IO, Iterable, Iterator, Optional, Union

import numpy as np
import torch

_HEADER = struct.Struct("<5i")
_DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16, "uint8": torch.uint8}
_NAMES = {v: k for k, v in _DTYPES.items()}
_ZSTD_MAGIC = b"\x28\xb5\x2f\xfd"
_ALIGN = 256


class RecordError(Exception):
    """A parameter record is cut short or malformed."""


def encode_record(scope: str, name: str, array: Union[np.ndarray, torch.Tensor]) -> bytes:
    """One record in the checkpoint format (numpy arrays or CPU tensors, any strides)."""
    t = torch.from_numpy(np.asarray(array, order="C")) if isinstance(array, np.ndarray) else array.detach().cpu()
    if t.dtype not in _NAMES:
        raise ValueError(f"encode_record: unsupported dtype {t.dtype}")
    data = t.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes() if t.numel() else b""
    s, n, d = scope.encode(), name.encode(), _NAMES[t.dtype].encode()
    return (_HEADER.pack(len(s), len(n), len(d), t.dim(), len(data)) + s + n + d +
            struct.pack(f"<{t.dim()}i", *t.shape) + data)


def _read_exact(stream: IO[bytes], size: int) -> bytes:
    chunks, left = [], size
    while left:
        chunk = stream.read(left)
        if not chunk:
            break
        chunks.append(chunk)
        left -= len(chunk)
    return b"".join(chunks)


def _read_header(stream: IO[bytes]):
    """(scope, name, dtype, shape, data bytes) of the next record, None at the end."""
    raw = _read_exact(stream, _HEADER.size)
    if not raw:
        return None
    if len(raw) < _HEADER.size:
        raise RecordError(f"record header cut short: {len(raw)} of {_HEADER.size} bytes")
    ls, ln, ld, ndim, nbytes = _HEADER.unpack(raw)
    if min(ls, ln, ld, ndim, nbytes) < 0:
        raise RecordError("record header has a negative length")
    meta_size = ls + ln + ld + 4 * ndim
    meta = _read_exact(stream, meta_size)
    if len(meta) < meta_size:
        raise RecordError(f"record payload cut short: {len(meta)} of {meta_size + nbytes} bytes")
    scope, name, dtype = meta[:ls].decode(), meta[ls:ls + ln].decode(), meta[ls + ln:ls + ln + ld].decode()
    shape = struct.unpack(f"<{ndim}i", meta[ls + ln + ld:])
    if dtype not in _DTYPES:
        raise RecordError(f"record {scope}/{name}: unsupported dtype {dtype!r}")
    tdtype = _DTYPES[dtype]
    expected = int(np.prod(shape, dtype=np.int64)) * torch.empty((), dtype=tdtype).element_size()
    if expected != nbytes:
        raise RecordError(f"record {scope}/{name}: shape {shape} of {dtype} is {expected} bytes, header says {nbytes}")
    return scope, name, tdtype, shape, nbytes


def read_records(stream: IO[bytes]) -> Iterator[tuple]:
    """(scope, name, CPU tensor) for every record of a byte stream (``xfold/params.py:67-96``)."""
    while True:
        head = _read_header(stream)
        if head is None:
            return
        scope, name, dtype, shape, nbytes = head
        data = _read_exact(stream, nbytes)
        if len(data) < nbytes:
            raise RecordError(f"record {scope}/{name} payload cut short: {len(data)} of {nbytes} bytes")
        if nbytes == 0:
            yield scope, name, torch.empty(shape, dtype=dtype)
        else:
            yield scope, name, torch.frombuffer(bytearray(data), dtype=torch.uint8).view(dtype).reshape(shape)


class ConcatenatedFiles(io.RawIOBase):
    """Read-only, seekable byte stream over several files in order (a checkpoint split
    into parts; records may cross part boundaries)."""

    def __init__(self, paths: Iterable[Union[str, Path]]):
        super().__init__()
        self._paths = [Path(p) for p in paths]
        if not self._paths:
            raise ValueError("ConcatenatedFiles: at least one file is required")
        self._sizes = [p.stat().st_size for p in self._paths]
        self._starts = np.concatenate([[0], np.cumsum(self._sizes)]).tolist()
        self._pos = 0
        self._handle, self._index = None, -1

    def readable(self) -> bool:
        return True

    def seekable(self) -> bool:
        return True

    def tell(self) -> int:
        return self._pos

    def seek(self, offset: int, whence: int = os.SEEK_SET) -> int:
        base = {os.SEEK_SET: 0, os.SEEK_CUR: self._pos, os.SEEK_END: self._starts[-1]}[whence]
        if base + offset < 0:
            raise ValueError("negative seek position")
        self._pos = base + offset
        return self._pos

    def readinto(self, buffer) -> int:
        view = memoryview(buffer).cast("B")
        done = 0
        while done < len(view) and self._pos < self._starts[-1]:
            index = int(np.searchsorted(self._starts, self._pos, side="right")) - 1
            if index != self._index:
                if self._handle is not None:
                    self._handle.close()
                self._handle, self._index = open(self._paths[index], "rb"), index
            local = self._pos - self._starts[index]
            self._handle.seek(local)
            want = min(len(view) - done, self._sizes[index] - local)
            got = self._handle.readinto(view[done:done + want])
            if not got:
                break
            done += got
            self._pos += got
        return done

    def close(self):
        if self._handle is not None:
            self._handle.close()
            self._handle = None
        super().close()


def _open(paths) -> IO[bytes]:
    paths = [paths] if isinstance(paths, (str, Path)) else list(paths)
    stream = io.BufferedReader(ConcatenatedFiles(paths), buffer_size=1 << 20)
    if stream.peek(4)[:4] == _ZSTD_MAGIC:
        try:
            import zstandard
        except ImportError as err:
            stream.close()
            raise RecordError("zstd-compressed checkpoint: install `zstandard` or decompress it first") from err
        data = zstandard.ZstdDecompressor().stream_reader(stream).read()
        stream.close()
        return io.BytesIO(data)
    return stream


def load_params(paths, device: Optional[Union[str, torch.device]] = None,
                staging_bytes: int = 64 << 20) -> dict:
    """``{"scope/name": tensor}`` for every record of the checkpoint file(s) ``paths``.

    ``device=None`` keeps CPU tensors. On a GPU the tensors are views of one device
    allocation filled through two pinned staging buffers of ``staging_bytes`` each (copies
    of one overlap the file reads into the other)."""
    device = torch.device(device) if device is not None else None
    if device is None or device.type == "cpu":
        with _open(paths) as stream:
            return {f"{s}/{n}": t for s, n, t in read_records(stream)}
    with _open(paths) as stream:
        index, offset = [], 0
        while True:                                   # pass 1: headers only
            head = _read_header(stream)
            if head is None:
                break
            index.append((head, offset, stream.tell()))
            offset += (head[4] + _ALIGN - 1) // _ALIGN * _ALIGN
            stream.seek(head[4], os.SEEK_CUR)
        arena = torch.empty(max(offset, 1), dtype=torch.uint8, device=device)
        # The arena comes from the caching allocator on the current stream: its block may
        # still be read by work queued there, so the copies start after that work.
        copy_stream = torch.cuda.Stream(device=device)
        copy_stream.wait_stream(torch.cuda.current_stream(device))
        staging = [torch.empty(staging_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        done = [None, None]
        slot, fill = 0, 0
        pending = []                                  # (arena offset, staging offset, bytes) of this slot

        def flush():
            nonlocal slot, fill, pending
            with torch.cuda.stream(copy_stream):
                for dst, src, nbytes in pending:
                    arena[dst:dst + nbytes].copy_(staging[slot][src:src + nbytes], non_blocking=True)
                event = torch.cuda.Event()
                event.record(copy_stream)
            done[slot] = event
            slot, fill, pending = slot ^ 1, 0, []
            if done[slot] is not None:
                done[slot].synchronize()              # the other buffer's copies have left it

        for (scope, name, dtype, shape, nbytes), dst, data_pos in index:   # pass 2: payloads
            stream.seek(data_pos)
            copied = 0
            while copied < nbytes:
                if fill == staging_bytes:
                    flush()
                take = min(nbytes - copied, staging_bytes - fill)
                view = memoryview(staging[slot].numpy())[fill:fill + take]
                got = 0
                while got < take:
                    n = stream.readinto(view[got:])
                    if not n:
                        raise RecordError(f"record {scope}/{name} payload cut short")
                    got += n
                pending.append((dst + copied, fill, take))
                fill += take
                copied += take
        if pending:
            flush()
        copy_stream.synchronize()
        torch.cuda.current_stream(device).wait_stream(copy_stream)
        params = {}
        for (scope, name, dtype, shape, nbytes), dst, _ in index:
            params[f"{scope}/{name}"] = arena[dst:dst + nbytes].view(dtype).reshape(shape)
        return params
