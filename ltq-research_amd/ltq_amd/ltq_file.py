"""The .ltq container of the quantizer's PACK output: tile packing and decoding on the GPU, file writing and
reading on the host.

Same names, arguments and file bytes as src/ltq_file.py:
  pack_slice / pack_slice_device   :79-96   four structure-of-arrays regions (codes, uncoded bit planes, lowest
                                             uncoded bit, gain indices), each on a 64-byte boundary, tiles by row
                                             group then 16-column block (position t = 16 r + c); HIP ltq_pack_slice
  decode_slice                     :119-147 the spec decoder; HIP ltq_unpack_slice
  assemble                         :150-156 W = H256(d q) * suh, d[m, b] = d_row[m] 2^(e[m, b] / 4)
  format_json / format_from_json   :40-50   the header's format description (lut and gains as exact floats)
  LtqWriter                        :163-225 writer: data region behind a reserved header, 64-byte aligned tensors,
                                             add_matrix with decode verification, finalize
  LtqFile                          :248-280 reader: header, memory-mapped tensors, decode_matrix
Ring records (rows of row tables): pack_rings_device, ring_bytes (src/ltq_format.py:42-50, 104-124).

File layout (a format, kept byte for byte): a 16-byte preamble (b"LTQ\0", uint32 version 1, uint64 header
reserve R, little endian), the UTF-8 JSON header (compact separators) space-padded to R bytes, then the data
region at 16 + R, a multiple of 4096. The header's "tensors" maps each name to {"dtype", "shape", "offset"}, the
offset relative to the data region and a multiple of 64; alignment gaps are zero bytes. A matrix p is five
tensors: p.ltq.slices (int32 [n, 4]: r0, r1, format index, byte offset in p.ltq.data), p.ltq.data (u8, the
packed row slices, each on a 64-byte boundary of the blob), p.ltq.d_row (f16 [M]), p.ltq.e (i8 [M, K / 256]) and
p.ltq.suh (f16 [K]).
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .formats import E_BITS, E_STEP, LtqFormat, exp2_table

MAGIC = b"LTQ\0"
VERSION = 1
TILE = 256
_PREAMBLE = struct.Struct("<4sIQ")
_DATA_ALIGN, _TENSOR_ALIGN = 4096, 64

# dtype code -> (element type of the stored bytes, torch dtype); bf16 is stored as its 16-bit pattern
DTYPES = {code: (np.dtype(npt), tt) for code, npt, tt in (
    ("f32", np.float32, torch.float32), ("f16", np.float16, torch.float16), ("bf16", np.uint16, torch.bfloat16),
    ("i32", np.int32, torch.int32), ("i8", np.int8, torch.int8), ("u8", np.uint8, torch.uint8))}
TORCH_TO_LTQ = {tt: code for code, (_, tt) in DTYPES.items()}
FRAC_NAMES = ("none", "d2", "d4")


def _round_up(n: int, a: int) -> int:
    return -(-n // a) * a


def _f32_list(a) -> list:
    """float32 values as Python floats (each float32 converts to a double exactly, so the JSON text names it
    uniquely and reads back to the same bits)."""
    return np.asarray(a, np.float32).astype(np.float64).tolist()


def format_json(f: LtqFormat) -> dict:
    """Header description of a format (key order is part of the file bytes)."""
    d = dict(name=f.name, K=f.K, frac=FRAC_NAMES[f.frac], masks=[int(m) for m in f.masks], h=f.h, sub=f.sub)
    d["lut"], d["gain"] = _f32_list(f.lut), _f32_list(f.gain_tab)
    return d


def format_from_json(d: dict) -> LtqFormat:
    """LtqFormat of a header description (the gain step is not stored: the gain table is)."""
    return LtqFormat(name=d["name"], K=int(d["K"]), frac=FRAC_NAMES.index(d["frac"]), masks=tuple(d["masks"]),
                     h=int(d["h"]), step=0.0, sub=int(d["sub"]), lut=np.asarray(d["lut"], np.float32),
                     gain_tab=np.asarray(d["gain"], np.float32))


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
    """W [M, K] = H256(d q) * suh over columns with d[m, b] = d_row[m] 2^(e[m, b] / 4) (src/ltq_file.py:150-156);
    the block factor is read from the shared exponent table (formats.exp2_table), as the quantizer's row scale
    reads it."""
    from . import rotation
    M, K = G.shape
    tab = torch.from_numpy(exp2_table(E_STEP, E_BITS)).to(G.device)
    scale = d_row.float().unsqueeze(1) * tab[e.long() + (1 << (E_BITS - 1))]
    Wq = (G.float().view(M, K // TILE, TILE) * scale.unsqueeze(2)).view(M, K)
    return rotation.fwht_inplace(Wq, block_size=TILE) * suh.float().unsqueeze(0)


def _host_bytes(t: torch.Tensor):
    """(dtype code, shape, raw bytes) of a tensor as the file stores it."""
    t = t.detach().to("cpu").contiguous()
    code = TORCH_TO_LTQ[t.dtype]
    arr = t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()
    return code, list(t.shape), arr.tobytes()


class LtqWriter:
    """Streams tensors into the data region of a new .ltq file; finalize(header) writes the preamble and the
    header into the reserved space. `tensors` is the catalog the header will carry, `quantized` the matrices
    added with add_matrix."""

    def __init__(self, path, formats, reserve: int = (64 << 20) - 16):
        if (_PREAMBLE.size + reserve) % _DATA_ALIGN:
            raise AssertionError(f"the data region must start on a {_DATA_ALIGN}-byte boundary (reserve {reserve})")
        self.path, self.reserve = Path(path), int(reserve)
        self.formats = list(formats)
        self.fmt_index = {f.name: i for i, f in enumerate(self.formats)}
        self.tensors: dict = {}
        self.quantized: list = []
        self._base = _PREAMBLE.size + self.reserve
        self._used = 0
        self._fh = open(self.path, "wb")
        self._fh.truncate(self._base)  # the reserved header space reads as zeros until finalize

    def _place(self, name: str, code: str, shape, payload) -> int:
        off = _round_up(self._used, _TENSOR_ALIGN)
        self._fh.seek(self._base + self._used)
        self._fh.write(bytes(off - self._used))
        self._fh.write(payload)
        self._used = off + len(payload)
        self.tensors[name] = {"dtype": code, "shape": [int(v) for v in shape], "offset": off}
        return off

    def add_tensor(self, name: str, t: torch.Tensor):
        self._place(name, *_host_bytes(t))

    def add_matrix(self, p: str, m: dict, verify: bool = True) -> int:
        """Writes PACK["matrix"] of the quantizer as the five tensors of matrix p; returns their payload bytes.
        The row slices are packed on the device into one blob; with verify, the spec decoder reads every slice
        back from the packed bytes and must give the quantizer's tile values G bit for bit."""
        M, K = m["idx"].shape
        table, chunks, used = [], [], 0
        for r0, r1, sp in m["row_slices"]:
            fi = self.fmt_index[sp]
            f = self.formats[fi]
            packed = pack_slice_device(m["idx"][r0:r1], m["gi"][r0:r1], f)
            if verify:
                dec = decode_slice(packed, r1 - r0, K, f, packed.device)
                want = m["G"][r0:r1].float().contiguous()
                n_bad = int((dec.view(torch.int32) != want.view(torch.int32)).sum())
                if n_bad:
                    raise RuntimeError(f"{p} [{r0}:{r1}] {sp}: decode disagrees with the quantizer in {n_bad} weights")
            start = _round_up(used, _TENSOR_ALIGN)
            if start > used:
                chunks.append(torch.zeros(start - used, dtype=torch.uint8, device=packed.device))
            chunks.append(packed)
            table.append([r0, r1, fi, start])
            used = start + packed.numel()
        blob = torch.cat(chunks).cpu().numpy().tobytes() if chunks else b""
        self.add_tensor(f"{p}.ltq.slices", torch.tensor(table, dtype=torch.int32))
        self._place(f"{p}.ltq.data", "u8", [len(blob)], blob)
        self.add_tensor(f"{p}.ltq.d_row", m["d_row"].to(torch.float16))
        self.add_tensor(f"{p}.ltq.e", m["e"].to(torch.int8))
        self.add_tensor(f"{p}.ltq.suh", m["suh"].to(torch.float16))
        self.quantized.append(p)
        return len(blob) + 16 * len(table) + 2 * M + M * (K // TILE) + 2 * K

    def finalize(self, header: dict):
        body = {**header, "tensors": self.tensors}
        text = json.dumps(body, ensure_ascii=False, separators=(",", ":")).encode("utf-8")
        if len(text) > self.reserve:
            raise AssertionError(f"header of {len(text)} B does not fit in the {self.reserve} B reserve")
        self._fh.seek(0)
        self._fh.write(_PREAMBLE.pack(MAGIC, VERSION, self.reserve))
        self._fh.write(text.ljust(self.reserve, b" "))
        self._fh.close()


class LtqFile:
    """Reader of an .ltq file: the parsed header, its formats, tensors mapped from the file, full matrix decode."""

    def __init__(self, path):
        self.path = Path(path)
        with open(self.path, "rb") as fh:
            pre = fh.read(_PREAMBLE.size)
            if len(pre) < _PREAMBLE.size:
                raise ValueError(f"{path}: too short for an .ltq preamble")
            magic, version, reserve = _PREAMBLE.unpack(pre)
            if magic != MAGIC or version != VERSION:
                raise ValueError(f"{path}: not an .ltq v{VERSION} file ({magic!r}, version {version})")
            self.header = json.loads(fh.read(reserve).decode("utf-8"))
        self.data_off = _PREAMBLE.size + reserve
        if self.data_off % _DATA_ALIGN:
            raise ValueError(f"{path}: data region at {self.data_off} is not {_DATA_ALIGN}-byte aligned")
        self.mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        self.formats = [format_from_json(d) for d in self.header["quantization"]["formats"]]

    def _entry(self, name: str):
        t = self.header["tensors"][name]
        np_t, torch_t = DTYPES[t["dtype"]]
        n = int(np.prod(t["shape"], dtype=np.int64)) * np_t.itemsize
        lo = self.data_off + int(t["offset"])
        return t, np_t, torch_t, lo, n

    def raw(self, name: str) -> memoryview:
        _, _, _, lo, n = self._entry(name)
        return memoryview(self.mm[lo:lo + n])

    def tensor(self, name: str) -> torch.Tensor:
        t, np_t, torch_t, lo, n = self._entry(name)
        arr = np.array(self.mm[lo:lo + n]).view(np_t).reshape(t["shape"])
        out = torch.from_numpy(arr)
        return out.view(torch.bfloat16) if torch_t == torch.bfloat16 else out

    def decode_matrix(self, p: str, device="cuda") -> torch.Tensor:
        """W [M, K] float32 as an engine reconstructs it from the file: every row slice decoded by the spec
        decoder, then assemble."""
        d_row = self.tensor(f"{p}.ltq.d_row").to(device)
        e = self.tensor(f"{p}.ltq.e").to(device)
        suh = self.tensor(f"{p}.ltq.suh").to(device)
        M, K = d_row.shape[0], suh.shape[0]
        blob = self.raw(f"{p}.ltq.data")
        G = torch.empty((M, K), dtype=torch.float32, device=device)
        for r0, r1, fi, off in self.tensor(f"{p}.ltq.slices").tolist():
            G[r0:r1] = decode_slice(blob[off:], r1 - r0, K, self.formats[fi], device)
        return assemble(G, d_row, e, suh)
