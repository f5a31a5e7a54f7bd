"""The .ltq container of the quantizer's PACK output: tile packing and decoding on the GPU, file writing and
reading on the host.

Mirrors src/ltq_file.py (same names, arguments and file layout):
  pack_slice / pack_slice_device   :79-96   four structure-of-arrays regions (codes, uncoded bit planes, lowest
                                             uncoded bit, gain indices), each on a 64-byte boundary, tiles by row
                                             group then 16-column block (position t = 16 r + c); HIP ltq_pack_slice
  decode_slice                     :119-147 the spec decoder; HIP ltq_unpack_slice
  assemble                         :150-156 W = H256(d q) * suh, d[m, b] = d_row[m] 2^(e[m, b] / 4)
  format_json / format_from_json   :40-50   the header's format description (lut and gains as exact floats)
  LtqWriter                        :163-225 data after a reserved header of 16 + reserve bytes (4096-aligned),
                                             tensors 64-byte aligned, add_matrix (with decode verification) and
                                             finalize (magic, version, reserve, space-padded JSON header)
  LtqFile                          :248-280 header parse, memory-mapped tensors, decode_matrix
Ring records (rows of row tables): pack_rings_device, ring_bytes (src/ltq_format.py:42-50, 104-124).
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .formats import LtqFormat

MAGIC = b"LTQ\0"
VERSION = 1
TILE = 256
DTYPES = {"f32": (np.float32, torch.float32), "f16": (np.float16, torch.float16), "bf16": (np.uint16, torch.bfloat16),
          "i32": (np.int32, torch.int32), "i8": (np.int8, torch.int8), "u8": (np.uint8, torch.uint8)}
TORCH_TO_LTQ = {v[1]: k for k, v in DTYPES.items()}
FRAC_NAMES = ["none", "d2", "d4"]


def _align(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def format_json(f: LtqFormat) -> dict:
    """Header description of a format; lut and gains as float32 values written exactly (repr of each float32)."""
    return {"name": f.name, "K": f.K, "frac": FRAC_NAMES[f.frac], "masks": [int(m) for m in f.masks], "h": f.h,
            "sub": f.sub, "lut": [float(v) for v in np.asarray(f.lut, np.float32)],
            "gain": [float(v) for v in np.asarray(f.gain_tab, np.float32)]}


def format_from_json(d: dict) -> LtqFormat:
    return LtqFormat(d["name"], d["K"], FRAC_NAMES.index(d["frac"]), tuple(d["masks"]), d["h"], 0.0, d["sub"],
                     np.asarray(d["lut"], np.float32), np.asarray(d["gain"], np.float32))


def slice_bytes(R: int, K: int, f: LtqFormat) -> int:
    n = _lib.lib().ltq_slice_bytes(R, K, f.K, f.frac, f.h, f.sub)
    if n < 0:
        raise ValueError(f"slice [{R}, {K}] cannot hold format {f.name} tiles (R and K must be multiples of 16)")
    return n


@torch.no_grad()
def pack_slice_device(idx: torch.Tensor, gi: torch.Tensor, f: LtqFormat) -> torch.Tensor:
    """Packed slice as a uint8 device tensor."""
    _lib.require_device(idx)
    R, K = idx.shape
    ix = idx.to(torch.int16)
    g = gi.to(torch.uint8)
    if ix.stride(1) != 1:
        ix = ix.contiguous()
    if g.stride(1) != 1:
        g = g.contiguous()
    n = slice_bytes(R, K, f)
    out = torch.empty(n, dtype=torch.uint8, device=idx.device)
    rc = _lib.lib().ltq_pack_slice(ix.data_ptr(), ix.stride(0), g.data_ptr(), g.stride(0), R, K, f.K, f.frac, f.h,
                                   f.sub, out.data_ptr(), n, _lib.stream_ptr())
    if rc != 0:
        raise RuntimeError(f"ltq_pack_slice: HIP error code {rc}" if rc > 0 else "ltq_pack_slice: rejected arguments")
    return out


def pack_slice(idx: torch.Tensor, gi: torch.Tensor, f: LtqFormat) -> bytes:
    """Row slice data [R, K] (label * U + u and gain index per position) -> bytes, as the reference returns."""
    return bytes(pack_slice_device(idx, gi, f).cpu().numpy().tobytes())


def ring_bytes(L: int, f: LtqFormat) -> int:
    """Bytes of one packed ring of L positions (src/ltq_format.py:48-50, `tile_bytes(L)`; scale excluded)."""
    n = _lib.lib().ltq_ring_bytes(L, f.K, f.frac, f.h, f.sub)
    if n < 0:
        raise ValueError(f"rings of {L} values cannot hold format {f.name} (L % 16 == 0, L % sub == 0, L <= 512)")
    return n


@torch.no_grad()
def pack_rings_device(idx: torch.Tensor, gi: torch.Tensor, f: LtqFormat) -> torch.Tensor:
    """Rings [n, L] of codes (label * U + u) and gain indices -> uint8 device tensor [n, ring_bytes(L)], each row
    the fields codes / planes / lsb / gains of src/ltq_format.py:104-124 back to back."""
    _lib.require_device(idx)
    n, L = idx.shape
    ix = idx.to(torch.int16)
    g = gi.to(torch.uint8)
    if ix.stride(1) != 1:
        ix = ix.contiguous()
    if g.stride(1) != 1:
        g = g.contiguous()
    rb = ring_bytes(L, f)
    out = torch.empty((n, rb), dtype=torch.uint8, device=idx.device)
    rc = _lib.lib().ltq_pack_rings(ix.data_ptr(), ix.stride(0), g.data_ptr(), g.stride(0), n, L, f.K, f.frac, f.h,
                                   f.sub, out.data_ptr(), out.numel(), _lib.stream_ptr())
    if rc != 0:
        raise RuntimeError(f"ltq_pack_rings: HIP error code {rc}" if rc > 0 else "ltq_pack_rings: rejected arguments")
    return out


@torch.no_grad()
def decode_slice(data, R: int, K: int, f: LtqFormat, device) -> torch.Tensor:
    """Unscaled slice values [R, K] (gain[g] * lut[label * U + u]) from the packed bytes (host bytes / memoryview or
    a uint8 device tensor), decoded on the device by the spec rules."""
    dev = torch.device(device)
    n = slice_bytes(R, K, f)
    if isinstance(data, torch.Tensor):
        raw = data.to(dev, torch.uint8).contiguous()
    else:
        raw = torch.frombuffer(bytearray(bytes(data[:n])), dtype=torch.uint8).to(dev)
    _lib.require_device(raw)
    lut = torch.as_tensor(np.asarray(f.lut, np.float32), device=dev)
    gains = torch.as_tensor(np.asarray(f.gain_tab, np.float32), device=dev) if f.h else None
    out = torch.empty((R, K), dtype=torch.float32, device=dev)
    m = (list(f.masks) + [0, 0, 0, 0])[:4]
    rc = _lib.lib().ltq_unpack_slice(raw.data_ptr(), raw.numel(), R, K, f.K, f.frac, f.h, f.sub, m[0], m[1], m[2], m[3],
                                     len(f.masks), lut.data_ptr(), gains.data_ptr() if gains is not None else None,
                                     out.data_ptr(), K, _lib.stream_ptr())
    if rc != 0:
        raise RuntimeError(f"ltq_unpack_slice: HIP error code {rc}" if rc > 0 else "ltq_unpack_slice: rejected arguments")
    return out


@torch.no_grad()
def assemble(G: torch.Tensor, d_row: torch.Tensor, e: torch.Tensor, suh: torch.Tensor) -> torch.Tensor:
    """W = H256(d q) * suh over columns, d[m, b] = d_row[m] 2^(e[m, b] / 4) (src/ltq_file.py:150-156)."""
    from . import rotation
    M, K = G.shape
    scale = d_row.float().unsqueeze(1) * torch.exp2(0.25 * e.float())
    W = (scale.unsqueeze(2) * G.view(M, K // TILE, TILE)).view(M, K)
    return rotation.fwht_inplace(W, block_size=TILE) * suh.float().unsqueeze(0)


class LtqWriter:
    """Writes tensors straight to the file behind a reserved header (data starts at 16 + reserve, a multiple of
    4096); `finalize` writes magic, version, reserve and the JSON header, space-padded to the reserve."""

    def __init__(self, path, formats, reserve: int = (64 << 20) - 16):
        assert (16 + reserve) % 4096 == 0
        self.path, self.reserve = Path(path), reserve
        self.formats = list(formats)
        self.fmt_index = {f.name: i for i, f in enumerate(self.formats)}
        self.f = open(self.path, "wb")
        self.f.write(bytes(16 + reserve))
        self.cur = 0
        self.tensors = {}
        self.quantized = []

    def _write(self, name: str, raw: bytes, dtype: str, shape, align: int = 64):
        pad = _align(self.cur, align) - self.cur
        if pad:
            self.f.write(bytes(pad))
            self.cur += pad
        self.tensors[name] = {"dtype": dtype, "shape": [int(v) for v in shape], "offset": self.cur}
        self.f.write(raw)
        self.cur += len(raw)

    def add_tensor(self, name: str, t: torch.Tensor):
        t = t.detach().cpu().contiguous()
        dt = TORCH_TO_LTQ[t.dtype]
        raw = t.view(torch.int16).numpy().tobytes() if t.dtype == torch.bfloat16 else t.numpy().tobytes()
        self._write(name, raw, dt, list(t.shape))

    def add_matrix(self, p: str, m: dict, verify: bool = True) -> int:
        """A matrix from PACK["matrix"] of the quantizer; returns the byte size of its fields. With verify, each
        slice decoded from the written bytes must equal the quantizer's tile values G bit for bit."""
        M, K = m["idx"].shape
        rows, data = [], bytearray()
        for r0, r1, sp in m["row_slices"]:
            f = self.formats[self.fmt_index[sp]]
            data += bytes(_align(len(data), 64) - len(data))
            rows.append([r0, r1, self.fmt_index[sp], len(data)])
            dev_bytes = pack_slice_device(m["idx"][r0:r1], m["gi"][r0:r1], f)
            if verify:
                G = m["G"][r0:r1]
                dec = decode_slice(dev_bytes, r1 - r0, K, f, G.device)
                bad = int((dec.view(torch.int32) != G.float().contiguous().view(torch.int32)).sum())
                if bad:
                    raise RuntimeError(f"{p} [{r0}:{r1}] {sp}: decode disagrees with the quantizer in {bad} weights")
            data += bytes(dev_bytes.cpu().numpy().tobytes())
        self.add_tensor(f"{p}.ltq.slices", torch.tensor(rows, dtype=torch.int32))
        self._write(f"{p}.ltq.data", bytes(data), "u8", [len(data)])
        self.add_tensor(f"{p}.ltq.d_row", m["d_row"].to(torch.float16))
        self.add_tensor(f"{p}.ltq.e", m["e"].to(torch.int8))
        self.add_tensor(f"{p}.ltq.suh", m["suh"].to(torch.float16))
        self.quantized.append(p)
        return len(data) + 16 * len(rows) + 2 * M + M * (K // TILE) + 2 * K

    def finalize(self, header: dict):
        header = dict(header, tensors=self.tensors)
        raw = json.dumps(header, ensure_ascii=False, separators=(",", ":")).encode("utf-8")
        assert len(raw) <= self.reserve, f"header of {len(raw)} B does not fit in the {self.reserve} B reserve"
        self.f.seek(0)
        self.f.write(MAGIC + struct.pack("<IQ", VERSION, self.reserve) + raw + b" " * (self.reserve - len(raw)))
        self.f.close()


class LtqFile:
    """Reader: header, memory-mapped tensors and the full decode of a matrix."""

    def __init__(self, path):
        with open(path, "rb") as fh:
            magic, (ver, H) = fh.read(4), struct.unpack("<IQ", fh.read(12))
            if magic != MAGIC or ver != VERSION:
                raise ValueError(f"{path}: not an .ltq v{VERSION} file ({magic!r}, version {ver})")
            self.header = json.loads(fh.read(H).decode("utf-8"))
        self.data_off = 16 + H
        if self.data_off % 4096:
            raise ValueError(f"{path}: data offset {self.data_off} is not 4096-aligned")
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        self.formats = [format_from_json(d) for d in self.header["quantization"]["formats"]]

    def raw(self, name: str) -> memoryview:
        t = self.header["tensors"][name]
        n = int(np.prod(t["shape"])) * np.dtype(DTYPES[t["dtype"]][0]).itemsize
        o = self.data_off + t["offset"]
        return memoryview(self.mm[o:o + n])

    def tensor(self, name: str) -> torch.Tensor:
        t = self.header["tensors"][name]
        np_dt, _ = DTYPES[t["dtype"]]
        arr = torch.from_numpy(np.frombuffer(self.raw(name), dtype=np_dt).copy()).reshape(t["shape"])
        return arr.view(torch.bfloat16) if t["dtype"] == "bf16" else arr

    def decode_matrix(self, p: str, device="cuda") -> torch.Tensor:
        """The matrix W [M, K] float32, as an engine reconstructs it."""
        d_row, e, suh = (self.tensor(f"{p}.ltq.{k}").to(device) for k in ("d_row", "e", "suh"))
        M, K = d_row.shape[0], suh.shape[0]
        data = self.raw(f"{p}.ltq.data")
        G = torch.empty((M, K), device=device)
        for r0, r1, fi, off in self.tensor(f"{p}.ltq.slices").tolist():
            G[r0:r1] = decode_slice(data[off:], r1 - r0, K, self.formats[fi], device)
        return assemble(G, d_row, e, suh)
