"""model.bin reader and writer (the reference's weight file format).

Reference: ModelLoader (include/model_loader.h, src/model_loader.cu:14-53).
Format, little-endian, offsets absolute from the start of the file:

    u32 count
    count x { u32 name_len; name bytes; u32 ndim; ndim x u32 dim; u64 offset; u64 bytes }
    tensor data: fp32 row-major, `bytes` bytes at `offset`

``ModelLoader`` parses the index once and loads a tensor straight into
pinned host memory and from there to the device, where weights stay
resident (the reference uploads every loaded tensor).  Errors raise
RuntimeError with the reference's messages: "cannot open model: <path>",
"truncated model.bin", "missing tensor: <name>", "tensor is not float32:
<name>", "truncated tensor: <name>".  ``write_model_bin`` writes the format
(tensor data 256-byte aligned); the reference ships no writer.
"""
from __future__ import annotations

import struct
from typing import Dict, Iterable, List, Tuple, Union

import numpy as np
import torch


class ModelLoader:
    def __init__(self, path: str):
        self.path = path
        self._entries: Dict[str, Tuple[Tuple[int, ...], int, int]] = {}
        self._staging = None
        try:
            f = open(path, "rb")
        except OSError:
            raise RuntimeError(f"cannot open model: {path}") from None
        with f:
            def field(fmt):
                n = struct.calcsize(fmt)
                b = f.read(n)
                if len(b) != n:
                    raise RuntimeError("truncated model.bin")
                return struct.unpack(fmt, b)

            (count,) = field("<I")
            for _ in range(count):
                (name_len,) = field("<I")
                name = f.read(name_len)
                if len(name) != name_len:
                    raise RuntimeError("truncated model.bin")
                (ndim,) = field("<I")
                shape = field(f"<{ndim}I") if ndim else ()
                offset, nbytes = field("<QQ")
                # the first entry of a name wins, as with the reference's map emplace
                self._entries.setdefault(name.decode("utf-8", "surrogateescape"), (tuple(shape), offset, nbytes))

    def has(self, name: str) -> bool:
        return name in self._entries

    def names(self) -> List[str]:
        return list(self._entries)

    def _entry(self, name: str):
        if name not in self._entries:
            raise RuntimeError(f"missing tensor: {name}")
        shape, offset, nbytes = self._entries[name]
        if nbytes != int(np.prod(shape, dtype=np.int64)) * 4:
            raise RuntimeError(f"tensor is not float32: {name}")
        return shape, offset, nbytes

    def load_numpy(self, name: str) -> np.ndarray:
        shape, offset, nbytes = self._entry(name)
        out = np.empty(shape, dtype=np.float32)
        with open(self.path, "rb") as f:
            f.seek(offset)
            if f.readinto(out.reshape(-1).view(np.uint8)) != nbytes:
                raise RuntimeError(f"truncated tensor: {name}")
        return out

    def load(self, name: str, device: Union[str, torch.device] = "cuda") -> torch.Tensor:
        """The tensor on `device` (fp32).  For a GPU the file is read into a
        grow-only pinned staging buffer of this loader, so that the upload is
        one DMA transfer without a pageable bounce."""
        shape, offset, nbytes = self._entry(name)
        dev = torch.device(device)
        if dev.type != "cuda":
            return torch.from_numpy(self.load_numpy(name)).to(dev)
        if self._staging is None or self._staging.numel() < nbytes:
            self._staging = torch.empty(max(nbytes, 1), dtype=torch.uint8, pin_memory=True)
        host = self._staging[:nbytes]
        with open(self.path, "rb") as f:
            f.seek(offset)
            if f.readinto(host.numpy()) != nbytes:
                raise RuntimeError(f"truncated tensor: {name}")
        out = torch.empty(shape, dtype=torch.float32, device=dev)
        out.view(-1).view(torch.uint8).copy_(host)  # synchronous: the staging buffer is reused
        return out

    def load_all(self, names: Iterable[str], device: Union[str, torch.device] = "cuda") -> List[torch.Tensor]:
        """Several tensors to a GPU with the file reads overlapped with the
        uploads: two pinned staging buffers, each upload an asynchronous copy
        on a side stream, a buffer refilled only after its previous upload
        has finished (its event)."""
        dev = torch.device(device)
        names = list(names)
        if dev.type != "cuda":
            return [self.load(n, dev) for n in names]
        entries = [self._entry(n) for n in names]
        cap = max([nb for _, _, nb in entries] + [1])
        bufs = [torch.empty(cap, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        done = [None, None]
        stream = torch.cuda.Stream(device=dev)
        outs = []
        with open(self.path, "rb") as f:
            for i, (name, (shape, offset, nbytes)) in enumerate(zip(names, entries)):
                k = i & 1
                if done[k] is not None:
                    done[k].synchronize()  # the upload that last read this buffer has finished
                host = bufs[k][:nbytes]
                f.seek(offset)
                if f.readinto(host.numpy()) != nbytes:
                    raise RuntimeError(f"truncated tensor: {name}")
                out = torch.empty(shape, dtype=torch.float32, device=dev)
                with torch.cuda.stream(stream):
                    out.view(-1).view(torch.uint8).copy_(host, non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(stream)
                done[k] = ev
                outs.append(out)
        stream.synchronize()
        torch.cuda.current_stream(dev).wait_stream(stream)
        return outs


def write_model_bin(path: str, tensors: Union[Dict[str, np.ndarray], Iterable[Tuple[str, np.ndarray]]],
                    align: int = 256) -> None:
    """Writes fp32 tensors in the model.bin format (index, then data at
    `align`-byte aligned offsets, in the given order)."""
    items = list(tensors.items() if isinstance(tensors, dict) else tensors)
    header = bytearray(struct.pack("<I", len(items)))
    sizes = [len(struct.pack("<I", 0)) + len(n.encode()) + 4 + 4 * np.asarray(a).ndim + 16 for n, a in items]
    pos = len(header) + sum(sizes)
    layout = []
    for name, a in items:
        a = np.asarray(a, dtype=np.float32)
        if not a.flags.c_contiguous:
            a = a.copy(order="C")
        pos = (pos + align - 1) // align * align
        layout.append((name, a, pos))
        pos += a.nbytes
    for name, a, off in layout:
        nb = name.encode()
        header += struct.pack("<I", len(nb)) + nb + struct.pack("<I", a.ndim)
        header += struct.pack(f"<{a.ndim}I", *a.shape) if a.ndim else b""
        header += struct.pack("<QQ", off, a.nbytes)
    with open(path, "wb") as f:
        f.write(header)
        for _, a, off in layout:
            f.seek(off)
            f.write(a.tobytes())
        f.truncate(pos if layout else len(header))


def moe_layer_tensors(layer: int, gate: np.ndarray, w1, w2, w3) -> Dict[str, np.ndarray]:
    """One MoE layer's tensors under the reference's names (src/layer.cu:44-47,
    94-100): model.layers.<i>.block_sparse_moe.gate.weight and
    ....experts.<e>.{w1,w2,w3}.weight."""
    base = f"model.layers.{layer}.block_sparse_moe"
    out = {f"{base}.gate.weight": gate}
    for e in range(len(w1)):
        for nm, w in (("w1", w1), ("w2", w2), ("w3", w3)):
            out[f"{base}.experts.{e}.{nm}.weight"] = w[e]
    return out


__all__ = ["ModelLoader", "write_model_bin", "moe_layer_tensors"]
