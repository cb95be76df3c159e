"""The `block_criterion` restore-swap name grammar (reference src/ress/scoring/criterion.py).

    base   := ["damage_"] "restore_swap" ["_iter" N]
    suffix := "_nowo" | "_wo" | "_bf16" | "_trackbest" | "_rf" NN | "_dc" NN | "_antiswap" | "_anti"

Suffixes may come in any order. `damage_` / `_nowo` select M = identity; `_rf`/`_dc` are
percentages; `_antiswap` maximises in the rounds, `_anti` also inverts the initial cut.
"""

import re
from dataclasses import dataclass

import torch

_SUFFIX = re.compile(r"_(nowo|wo|bf16|trackbest|rf\d+|dc\d+|antiswap|anti)$")
_BASE = re.compile(r"^(damage_)?restore_swap(?:_iter(\d+))?$")


@dataclass
class RestoreSwapSpec:
    """Arguments of restore_swap_rank_by parsed from a criterion name
    (reference criterion.py:53-77)."""

    n_iters: int = 1
    use_wo: bool = True
    track_best: bool = False
    big_dtype: torch.dtype | None = None
    restore_frac: float = 0.5
    maximize: bool = False
    invert_cut: bool = False
    decay: float = 0.5


def _split(name):
    core, suffixes = name, []
    while True:
        m = _SUFFIX.search(core)
        if m is None:
            return core, suffixes
        suffixes.append(m.group(1))
        core = core[:m.start()]


def is_restore_swap(block_criterion):
    return _BASE.match(_split(block_criterion)[0]) is not None


def parse_restore_swap(block_criterion):
    core, suffixes = _split(block_criterion)
    m = _BASE.match(core)
    if m is None:
        raise ValueError(f"not a restore-swap block_criterion: {block_criterion!r}")
    spec = RestoreSwapSpec(n_iters=int(m.group(2)) if m.group(2) else 1, use_wo=m.group(1) is None)
    for s in suffixes:
        if s == "nowo":
            spec.use_wo = False
        elif s == "wo":
            spec.use_wo = True
        elif s == "trackbest":
            spec.track_best = True
        elif s == "antiswap":
            spec.maximize = True
        elif s == "anti":
            spec.maximize = True
            spec.invert_cut = True
        elif s.startswith("rf"):
            spec.restore_frac = int(s[2:]) / 100.0
        elif s.startswith("dc"):
            spec.decay = int(s[2:]) / 100.0
        else:
            spec.big_dtype = torch.bfloat16
    return spec
