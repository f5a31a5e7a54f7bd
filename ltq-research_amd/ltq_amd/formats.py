"""TCQ format definitions: TCQ_CONFIG, the .ltq tile format description and the format menus.

Mirrors src/liqk_v2.py:779-840 (TCQ_CONFIG construction), src/ltq_format.py:16-66 (NU, TILE, MASK_M,
LtqFormat, load_formats) and src/equal_bpw.py:42-75 (SETS menus). The trained tables themselves are data,
extracted unchanged into data/tcq_tables.json by tests/golden/make_tables.py.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from statistics import NormalDist
from pathlib import Path
from typing import Dict

import numpy as np

QK_K = 256            # weights per tile / per row block (src/iqk_format.py:23)
SUBBLOCK_SIZE = 16    # weights per gain index (src/iqk_format.py:24)
NUM_SUBBLOCKS = QK_K // SUBBLOCK_SIZE
NU = 10               # trellis memory: state = last 10 code bits (src/ltq_format.py:16)
TILE = 256
MASK_M = 359          # primary Ungerboeck label mask (src/ltq_format.py:18)

_TABLES = json.loads((Path(__file__).resolve().parent / "data" / "tcq_tables.json").read_text())


def _build_config() -> Dict[str, dict]:
    cfg: Dict[str, dict] = {k: dict(v) for k, v in _TABLES["base"].items()}
    # R variants: one d per row + 5-bit block exponent, trellis state carried between tiles (liqk_v2.py:826-828)
    for k, sc in ((2, 1.05), (3, 1.15), (4, 1.25)):
        cfg[f"TCQ{k}R"] = dict(cfg[f"TCQ{k}"], row_scale=True, carry=True, scale=sc)
    for name, v in _TABLES["variants"].items():
        v = dict(v)
        parent = v.pop("parent")
        cfg[name] = dict(cfg[parent], **v)
    # half-integer R formats: alternating K / K+1 tile rows (liqk_v2.py:813-821)
    for k in (2, 3):
        cfg[f"TCQ{k}5R"] = {"K": k, "K_hi": k + 1, "nu": 10, "m": 359, "h": 1, "row_scale": True, "carry": True,
                            "scale": 1.0, "lo": f"TCQ{k}R", "hi": f"TCQ{k + 1}R"}
    # night-2 tail-biting formats with extended labels (liqk_v2.py:834-840)
    xs = _TABLES["x_scale"]
    for name, t in _TABLES["x_tables"].items():
        cfg[name] = {"K": t["K"], "nu": 10, "m": 359, "h": t["h"], "step": t["step"], "lut": t["lut"],
                     "sub": t.get("sub", SUBBLOCK_SIZE), "pp": t.get("pp", False), "scale": xs.get(name, 1.0),
                     "m_extra": tuple(t["m_extra"]), "row_scale": True, "tb": True,
                     **({"n_cand": 4} if t["h"] > 2 else {})}
    # the MoE expert format: K=3 D4 with 16-subset labels (the Y family's masks 40, 475), a
    # 3-bit gain header searched over 4 candidates; no trained table exists in the reference, so its table is
    # the closed-form start of table training (src/universal_bench.py:91-94)
    cfg["TCQ275Y3"] = {"K": 3, "nu": 10, "m": 359, "h": 3, "step": 0.15, "lut": closed_form_lut(3, (40, 475)),
                       "sub": SUBBLOCK_SIZE, "pp": 2, "scale": 1.1, "m_extra": (40, 475), "row_scale": True,
                       "tb": True, "n_cand": 4}
    return cfg


def closed_form_lut(K: int, m_extra: tuple, spread: float = 1.0) -> list:
    """The table-training start as a list of float32 values: entry lb * U + u = the (u * nl + lb)-th of the nl * U
    midpoint quantiles (k + 1/2) / (nl U) of N(0, spread^2), in float64 (the same values as
    tables.closed_form_table)."""
    nl, U = 4 << len(m_extra), 1 << (K - 1)
    n = nl * U
    nd = NormalDist(0.0, spread)
    grid = np.array([nd.inv_cdf((k + 0.5) / n) for k in range(n)], dtype=np.float64).astype(np.float32)
    return [float(grid[u * nl + lb]) for lb in range(nl) for u in range(U)]


TCQ_CONFIG: Dict[str, dict] = _build_config()
TCQ_X_SCALE: Dict[str, float] = dict(_TABLES["x_scale"])

# format menus (src/equal_bpw.py:47-75)
_X5 = ["TCQ2X0", "TCQ2X", "TCQ3X1", "TCQ3X", "TCQ4X1", "TCQ4X2", "TCQ4X", "TCQ5X3", "TCQ5X"]
SETS = {
    "TCQX": ["TCQ2X0", "TCQ2X", "TCQ3X1", "TCQ3X", "TCQ4X1", "TCQ4X2", "TCQ4X"],
    "TCQX5": list(_X5),
    "TCQP": _X5 + ["TCQ4W2", "TCQ4W3", "TCQ25X", "TCQ35X1", "TCQ35X", "TCQ45X"],
    "TCQPQ": _X5 + ["TCQ4W2", "TCQ4W3", "TCQ25X", "TCQ35X1", "TCQ35X", "TCQ45X", "TCQ275X", "TCQ275X2", "TCQ375X",
                    "TCQ475X"],
    "TCQPQE": _X5 + ["TCQ4W2", "TCQ4W3", "TCQ25X", "TCQ35X1", "TCQ35X", "TCQ45X", "TCQ275X", "TCQ275X2", "TCQ375X",
                     "TCQ475X", "TCQ225X", "TCQ325X", "TCQ425X"],
}

FRAC_RATE = {0: 0.0, 1: 0.5, 2: 0.25, 3: 0.75}

# row-scale block exponent (src/liqk_v2.py:943-946): d = d_row * 2^(E_STEP * e), e in [-2^(E_BITS-1), 2^(E_BITS-1))
E_STEP, E_BITS = 0.25, 5


def exp2_table(e_step: float = E_STEP, e_bits: int = E_BITS) -> np.ndarray:
    """float32 [2^e_bits]: entry k = 2^(e_step * (k - 2^(e_bits-1))), evaluated in float64 and rounded once to
    float32. The one table of block-exponent factors: the quantizer's row scale, the PACK tail, the .ltq decoder
    (assemble) and the CPU oracle all read it, so the scale d of a block is the same bits everywhere. For the
    .ltq exponent (e_step 0.25, 5 bits) it equals torch's float32 exp2(0.25 * e) entry for entry."""
    half = 1 << (e_bits - 1)
    return np.array([2.0 ** (e_step * (k - half)) for k in range(2 * half)], dtype=np.float32)


@dataclass(frozen=True)
class LtqFormat:
    """One .ltq tile format (src/ltq_format.py:21-54): K bits/weight before the fractional mode, frac (0 none,
    1 D2, 2 D4), label masks, gain header bits h, gain step, weights per gain index, LUT and the explicit gain
    table (stored in the file, so that decoders use the quantizer's exact values)."""
    name: str
    K: int
    frac: int
    masks: tuple
    h: int
    step: float
    sub: int
    lut: np.ndarray
    gain_tab: np.ndarray

    @property
    def n_labels(self) -> int:
        return 2 ** len(self.masks) * 2

    @property
    def U(self) -> int:
        return 1 << (self.K - 1)

    def lsb_words(self, L: int = TILE) -> int:
        return ({0: L, 1: L // 2, 2: 3 * L // 4}[self.frac] + 15) // 16

    def gain_words(self, L: int = TILE) -> int:
        return (L // self.sub * self.h + 15) // 16

    def tile_bytes(self, L: int = TILE) -> int:
        return 2 * (L // 16 + L // 16 * (self.K - 2) + (self.lsb_words(L) if self.K > 1 else 0) + self.gain_words(L))

    def bpw(self, k_in: int) -> float:
        return self.tile_bytes() * 8 / TILE + 8 / 256 + 16 / k_in


def make_format(name: str) -> LtqFormat:
    from .tcq_proto import make_gains
    c = TCQ_CONFIG[name]
    return LtqFormat(name, c["K"], int(c.get("pp", 0)), (c["m"],) + tuple(c.get("m_extra", ())), c["h"],
                     float(c["step"]), c.get("sub", 16), np.asarray(c["lut"], dtype=np.float32),
                     make_gains(c["h"], c["step"], "cpu").numpy())


def load_formats(menu) -> Dict[str, LtqFormat]:
    """Formats of a menu (src/ltq_format.py:57-66); gains are evaluated on the CPU (the reference uses the
    quantizing device, whose pow rounding may differ; the .ltq header stores the table explicitly)."""
    return {name: make_format(name) for name in menu}
