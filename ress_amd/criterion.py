"""The restore-swap `block_criterion` names (the grammar of the reference's
src/ress/scoring/criterion.py:3-7,96-124).

    name   := ["damage_"] "restore_swap" ["_iter" N] { suffix }
    suffix := "_nowo" | "_wo" | "_bf16" | "_trackbest" | "_rf" NN | "_dc" NN | "_antiswap" | "_anti"

Semantics kept from the reference: suffixes may come in any order; when two suffixes set
the same field the leftmost one wins; `damage_` and `_nowo` both mean M = identity;
`_rf`/`_dc` are percentages of restore_frac / decay; `_antiswap` maximises J in the
rounds and `_anti` also inverts the initial cut.

The parser splits the name on "_" and reads suffix tokens off the right end against a
table, then checks that what remains is the base; no regular expressions.
"""

from dataclasses import dataclass, fields

import torch


@dataclass
class RestoreSwapSpec:
    """Keyword arguments of restore_swap_rank_by named by a criterion
    (reference criterion.py:53-77 defaults)."""

    n_iters: int = 1
    use_wo: bool = True
    track_best: bool = False
    big_dtype: torch.dtype | None = None
    restore_frac: float = 0.5
    maximize: bool = False
    invert_cut: bool = False
    decay: float = 0.5


# suffix token -> the fields it sets
_FLAG_TOKENS = {
    "nowo": {"use_wo": False},
    "wo": {"use_wo": True},
    "bf16": {"big_dtype": torch.bfloat16},
    "trackbest": {"track_best": True},
    "antiswap": {"maximize": True},
    "anti": {"maximize": True, "invert_cut": True},
}
# percentage suffixes: token prefix -> field (value = digits / 100)
_PERCENT_TOKENS = {"rf": "restore_frac", "dc": "decay"}
_SPEC_FIELDS = {f.name for f in fields(RestoreSwapSpec)}


def _digits(s):
    return s != "" and s.isdecimal()


def _suffix_fields(token):
    """The fields a suffix token sets, or None if the token is not a suffix."""
    if token in _FLAG_TOKENS:
        return _FLAG_TOKENS[token]
    for prefix, field in _PERCENT_TOKENS.items():
        if token.startswith(prefix) and _digits(token[len(prefix):]):
            return {field: int(token[len(prefix):]) / 100.0}
    return None


def _tokenize(block_criterion):
    """(base tokens, suffix field updates ordered right to left) or None if the name is not
    a restore-swap criterion."""
    if not isinstance(block_criterion, str):
        return None
    tokens = block_criterion.split("_")
    updates = []
    while tokens:
        upd = _suffix_fields(tokens[-1])
        if upd is None:
            break
        updates.append(upd)
        tokens.pop()
    base = tokens[1:] if tokens[:1] == ["damage"] else tokens
    if base[:2] != ["restore", "swap"]:
        return None
    rest = base[2:]
    if rest and not (len(rest) == 1 and rest[0].startswith("iter") and _digits(rest[0][4:])):
        return None
    return tokens, updates


def is_restore_swap(block_criterion):
    """True if `block_criterion` names a restore-swap ranking (reference criterion.py:80-82)."""
    return _tokenize(block_criterion) is not None


def parse_restore_swap(block_criterion):
    """RestoreSwapSpec for a restore-swap criterion name; ValueError otherwise
    (reference criterion.py:96-124)."""
    parsed = _tokenize(block_criterion)
    if parsed is None:
        raise ValueError(f"not a restore-swap block_criterion: {block_criterion!r}")
    base, updates = parsed
    spec = RestoreSwapSpec(use_wo=base[0] != "damage")
    tail = base[-1]
    if tail.startswith("iter"):
        spec.n_iters = int(tail[4:])
    # updates run right to left, so the leftmost suffix that sets a field is applied last
    for upd in updates:
        for field, value in upd.items():
            assert field in _SPEC_FIELDS
            setattr(spec, field, value)
    return spec
