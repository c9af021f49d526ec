"""Recognising an svdq checkpoint inside a model snapshot, and whether this build can serve it.

The reference tags a nunchaku single-file checkpoint by its safetensors
``__metadata__`` (``src/gen_worker/models/svdq.py:58-129``): a
``quantization_config`` (JSON) whose ``method`` is ``svdquant``, a
``model_class`` named ``Nunchaku…``, the weight precision from
``quantization_config.weight.dtype`` (fp4 / int4) and the rank; it looks in
the denoiser component folders first, then at the snapshot root, and refuses
what it cannot serve with typed errors. This build serves both packagings:
int4 natively on the int4-g64 kernels (where the reference refuses,
``models/svdq.py:30-37``) and fp4 (block-16 e4m3 micro-scales,
``svdq_fp4``) folded to bf16 or, in the blockwise mode, with the reference's
fp4 numerics.

``load_svdq_artifact`` is the routing: detect, check, then load the file into
a caller-built module skeleton with the process's qualified lane
(``svdq_checkpoint.load_svdq_checkpoint``).
"""

from __future__ import annotations

import json
import logging
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Dict, Optional

logger = logging.getLogger(__name__)

SVDQ_METHOD = "svdquant"
DENOISER_DIRS = ("transformer", "unet", "transformer_2", "dit")   # snapshot folders that hold a denoiser
HEADER_LIMIT = 100 << 20   # the reference's MAX_HEADER_BYTES (models/safetensors_header.py:11): a larger
# declared header is treated as unreadable, never allocated


class SvdqArtifactError(RuntimeError):
    """Typed refusal of a detected svdq artifact."""


class SvdqPrecisionUnsupported(SvdqArtifactError):
    """The artifact's weight precision has no decoder / kernels in this build."""


@dataclass(frozen=True)
class SvdqArtifact:
    component: str          # the folder it was found in ("" at the root or for a bare file)
    file: Path
    model_class: str        # as stored (``Nunchaku…``)
    precision: str          # "int4" or "fp4"
    rank: int
    lowrank_quant: Optional[str]   # the declared low-rank scheme, None when the file declares none

    @property
    def denoiser_class(self) -> str:
        """The model class without nunchaku's prefix (the name the adaLN split table uses)."""
        return self.model_class[len("Nunchaku"):] if self.model_class.startswith("Nunchaku") else self.model_class


def read_safetensors_metadata(path: Path | str) -> Dict[str, Any]:
    """The ``__metadata__`` block of a safetensors file (8-byte little-endian header length, then the JSON
    header); {} for a file that is not readable as safetensors."""
    try:
        with open(path, "rb") as fh:
            head = fh.read(8)
            if len(head) != 8:
                return {}
            (length,) = struct.unpack("<Q", head)
            if not 0 < length <= HEADER_LIMIT:
                return {}
            header = json.loads(fh.read(length))
    except (OSError, ValueError):
        return {}
    meta = header.get("__metadata__") if isinstance(header, dict) else None
    return meta if isinstance(meta, dict) else {}


def _as_dict(value: Any) -> dict:
    if isinstance(value, dict):
        return value
    if isinstance(value, str):
        try:
            parsed = json.loads(value)
        except ValueError:
            return {}
        return parsed if isinstance(parsed, dict) else {}
    return {}


def artifact_of_file(path: Path | str, component: str = "") -> Optional[SvdqArtifact]:
    """The svdq artifact a safetensors file declares, or None for any other file."""
    meta = read_safetensors_metadata(path)
    qc = _as_dict(meta.get("quantization_config"))
    if str(qc.get("method") or "") != SVDQ_METHOD:
        return None
    model_class = str(meta.get("model_class") or "")
    if not model_class.startswith("Nunchaku"):
        return None
    dtype = str(_as_dict(qc.get("weight")).get("dtype") or "").lower()
    precision = "fp4" if "fp4" in dtype else "int4" if "int4" in dtype else ""
    if not precision:
        logger.warning("svdq artifact %s: unrecognised weight dtype %r; not treated as svdq", path, dtype)
        return None
    lowrank = meta.get("lowrank_quant")
    try:
        rank = int(qc.get("rank") or 0)
    except (TypeError, ValueError):
        rank = 0
    return SvdqArtifact(component, Path(path), model_class, precision, rank,
                        str(lowrank) if lowrank is not None else None)


def detect_svdq_artifact(model_path: Path | str) -> Optional[SvdqArtifact]:
    """The svdq checkpoint of a snapshot: a bare ``.safetensors`` file, else the first svdq-tagged file (by
    name) in the denoiser folders in ``DENOISER_DIRS`` order, else at the snapshot root."""
    root = Path(model_path)
    if root.is_file():
        return artifact_of_file(root) if root.suffix == ".safetensors" else None
    if not root.is_dir():
        return None
    places = [(d, root / d) for d in DENOISER_DIRS] + [("", root)]
    for component, folder in places:
        if not folder.is_dir():
            continue
        for f in sorted(folder.glob("*.safetensors")):
            art = artifact_of_file(f, component)
            if art is not None:
                return art
    return None


def check_svdq_servable(art: SvdqArtifact) -> None:
    """Raise the typed refusal for an artifact this build cannot serve (nothing for the int4 and fp4
    packagings with a known low-rank scheme)."""
    if art.precision not in ("int4", "fp4"):
        raise SvdqPrecisionUnsupported(f"{art.file} is svdq-{art.precision}: this build decodes the int4 group-64 "
                                       f"and the fp4 block-16 svdq packagings")
    from .svdq_checkpoint import LOWRANK_SCHEMES

    if art.lowrank_quant not in (None, "bf16") and art.lowrank_quant not in LOWRANK_SCHEMES:
        raise SvdqArtifactError(f"{art.file} declares lowrank_quant={art.lowrank_quant!r}, not one of bf16, "
                                f"{', '.join(LOWRANK_SCHEMES)}")


def load_svdq_artifact(model_path: Path | str, model: Any, *, device: Any = "cuda", lane: Optional[str] = None,
                       adanorm_splits: Optional[Dict[str, int]] = None, fp4_mode: Optional[str] = None) -> dict:
    """Detect the snapshot's svdq checkpoint, refuse what this build cannot serve, and load it into ``model``
    (a module skeleton whose names match the checkpoint's): int4 linears by ``lane``, fp4 linears by
    ``fp4_mode`` ("dense" by default, "blockwise"). Returns the loader's counts plus the artifact."""
    from .svdq_checkpoint import load_svdq_checkpoint

    art = detect_svdq_artifact(model_path)
    if art is None:
        raise SvdqArtifactError(f"{model_path}: no svdq checkpoint (no safetensors file declares "
                                f"quantization_config.method = {SVDQ_METHOD!r} with a Nunchaku model_class)")
    check_svdq_servable(art)
    logger.info("svdq: %s %s rank %d (%s), low-rank branch %s", art.precision, art.model_class, art.rank,
                art.file.name, art.lowrank_quant or "bf16")
    counts = load_svdq_checkpoint(art.file, model, model_class=art.denoiser_class, adanorm_splits=adanorm_splits,
                                  device=device, lane=lane, lowrank_quant=art.lowrank_quant or "bf16",
                                  fp4_mode=fp4_mode, precision=art.precision)
    counts["artifact"] = art
    return counts


__all__ = [
    "DENOISER_DIRS", "SVDQ_METHOD", "SvdqArtifact", "SvdqArtifactError", "SvdqPrecisionUnsupported",
    "artifact_of_file", "check_svdq_servable", "detect_svdq_artifact", "load_svdq_artifact",
    "read_safetensors_metadata",
]
