"""On-disk format of packed ternary Block-ELL weights (version 1).

A file is a safetensors file (no pickled code: loading runs nothing from the file).  For every
weight ``<name>`` it holds three tensors:

  ``<name>.packed``       int32 [R, K, B, B/16]  word (r, k, D, e) packs the 16 codes of
                          t[r, k, 16e + i, D] (tile [B_in, B_out]; D = output column, 16e + i =
                          input row); the 2-bit code of i sits at bit 8*(i % 4) + 2*(i // 4), so
                          ``(word >> 2q) & 0x03030303`` gives the codes of i = 4q..4q+3 in bytes
                          0..3.  Codes: 0b00 = 0, 0b01 = +1, 0b11 = -1; 0b10 is invalid.
  ``<name>.scales``       float32 [R, K]  the tile's absmean scale: weight = scales[r, k] * t
  ``<name>.col_indices``  int32 [R, K]    input column block of each tile, -1 = dead slot

and the header metadata (strings): ``format`` = ``lbk-ternary-block-ell``, ``version`` = ``1``,
``weights`` = JSON list of the names, ``B`` = JSON object name -> tile size, optional
``in_features`` = JSON object name -> C*B, and any caller entries under ``user.<key>``.

``load_ternary`` checks the header, every shape and dtype, the column range when
``in_features`` is present, and every code (on the GPU, ``lbk_ternary_check_codes``) before it
returns the weights.  B is 16, 32 or 64.
"""

from __future__ import annotations

import ctypes as C
import json

import torch

from .. import abi as A

TERNARY_FORMAT = "lbk-ternary-block-ell"
TERNARY_VERSION = "1"


def check_ternary_codes(packed: torch.Tensor) -> int:
    """Number of 2-bit fields holding the invalid code 0b10 (counted on the GPU)."""
    if not packed.is_cuda:
        raise RuntimeError("check_ternary_codes runs on the GPU; got a CPU tensor")
    p = packed.contiguous()
    if p.dtype != torch.int32:
        raise TypeError("packed ternary words are int32")
    bad = torch.empty(1, dtype=torch.int32, device=p.device)
    st = C.c_void_p(torch.cuda.current_stream(p.device).cuda_stream)
    A.check(A.load().lbk_ternary_check_codes(C.c_void_p(p.data_ptr()), p.numel(), C.c_void_p(bad.data_ptr()), st),
            "ternary_check_codes")
    return int(bad.item())


def _parts(w):
    if isinstance(w, (tuple, list)):
        return tuple(w)
    return w.packed, w.scales, w.col_indices


def save_ternary(path: str, weights: dict, in_features: dict | None = None, metadata: dict | None = None) -> None:
    """Write ``{name: TernaryBlockELLWeight or (packed, scales, col_indices)}`` to ``path``."""
    from safetensors.torch import save_file
    tensors, tiles = {}, {}
    for name, w in weights.items():
        if "." in name and name.rsplit(".", 1)[1] in ("packed", "scales", "col_indices"):
            raise ValueError(f"weight name {name!r} ends in a reserved suffix")
        packed, scales, cols = _parts(w)
        R, K, B, E = packed.shape
        if packed.dtype != torch.int32 or E * 16 != B or B not in (16, 32, 64):
            raise ValueError(f"{name}: packed must be int32 [R, K, B, B/16] with B in 16/32/64")
        tensors[f"{name}.packed"] = packed.detach().contiguous().cpu()
        tensors[f"{name}.scales"] = scales.detach().float().contiguous().cpu()
        tensors[f"{name}.col_indices"] = cols.detach().to(torch.int32).contiguous().cpu()
        tiles[name] = B
    meta = {"format": TERNARY_FORMAT, "version": TERNARY_VERSION, "weights": json.dumps(list(weights)),
            "B": json.dumps(tiles)}
    if in_features:
        meta["in_features"] = json.dumps({k: int(v) for k, v in in_features.items()})
    for k, v in (metadata or {}).items():
        meta[f"user.{k}"] = str(v)
    save_file(tensors, path, metadata=meta)


def load_ternary(path: str, device="cuda", as_modules: bool = True):
    """Read a file written by ``save_ternary``; returns ``(weights, metadata)`` where weights maps
    name -> ``TernaryBlockELLWeight`` (or the ``(packed, scales, col_indices)`` triple)."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != TERNARY_FORMAT:
            raise ValueError(f"{path}: not a {TERNARY_FORMAT} file")
        if meta.get("version") != TERNARY_VERSION:
            raise ValueError(f"{path}: unsupported version {meta.get('version')!r}")
        names = json.loads(meta["weights"])
        tiles = json.loads(meta["B"])
        inf = json.loads(meta.get("in_features", "{}"))
        keys = set(f.keys())
        raw = {}
        for n in names:
            want = [f"{n}.packed", f"{n}.scales", f"{n}.col_indices"]
            if any(k not in keys for k in want):
                raise ValueError(f"{path}: weight {n!r} incomplete")
            raw[n] = [f.get_tensor(k) for k in want]
    out = {}
    for n, (packed, scales, cols) in raw.items():
        B = int(tiles[n])
        if packed.dtype != torch.int32 or packed.dim() != 4 or packed.shape[2] != B or packed.shape[3] * 16 != B:
            raise ValueError(f"{n}: packed has shape {tuple(packed.shape)} / {packed.dtype}, expected [R, K, {B}, "
                             f"{B // 16}] int32")
        R, K = packed.shape[:2]
        if scales.dtype != torch.float32 or tuple(scales.shape) != (R, K):
            raise ValueError(f"{n}: scales must be float32 [{R}, {K}]")
        if cols.dtype != torch.int32 or tuple(cols.shape) != (R, K):
            raise ValueError(f"{n}: col_indices must be int32 [{R}, {K}]")
        if n in inf:
            Cb = int(inf[n]) // B
            if bool(((cols >= Cb) | (cols < -1)).any()):
                raise ValueError(f"{n}: column index outside [-1, {Cb})")
        packed, scales, cols = packed.to(device), scales.to(device), cols.to(device)
        bad = check_ternary_codes(packed)
        if bad:
            raise ValueError(f"{n}: {bad} invalid 2-bit codes (0b10)")
        if as_modules:
            from ..layers.ternary import TernaryBlockELLWeight
            out[n] = TernaryBlockELLWeight(packed, scales, cols)
        else:
            out[n] = (packed, scales, cols)
    user = {k[5:]: v for k, v in meta.items() if k.startswith("user.")}
    return out, user
