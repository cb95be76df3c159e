"""The device's bf16 rounding against the rule the oracle states (round to nearest even, NaNs
made quiet with (u >> 16) | 0x40), over every fp32 bit pattern.

Every kernel rounds fp32 to bf16 with the gfx950 conversion instruction (round_bf16 in
csrc/common.h); the oracle (oracle/ress_oracle.c) states the rule as integer arithmetic on
the bits, and that rule is pinned against torch's .to(bfloat16) on the CPU. This checks that
the instruction and the rule agree on all 2^32 inputs, subnormals, infinities and NaNs
included, through ress_bf16_selfcheck."""

import pytest
import torch

from ress_amd import _lib

pytestmark = pytest.mark.gpu


def _check(first, count, dev):
    out = torch.tensor([0, -1], dtype=torch.int64, device=dev)  # {mismatches, lowest pattern}
    _lib.call("ress_bf16_selfcheck", first, count, _lib.ptr(out), _lib.stream_handle(dev))
    torch.cuda.synchronize()
    bad, low = out.cpu().tolist()
    return bad, low & 0xFFFFFFFF


def test_device_bf16_rounding_matches_the_rule_on_every_fp32(dev):
    bad, low = _check(0, 1 << 32, dev)
    assert bad == 0, f"{bad} fp32 patterns round differently, the lowest {low:#010x}"


def test_selfcheck_counts_a_partial_range(dev):
    # the sweep's own bookkeeping: an empty range reports nothing, a range ending at the top
    # pattern wraps nowhere and agrees too
    assert _check(0, 0, dev) == (0, 0xFFFFFFFF)
    assert _check(0xFFFF0000, 1 << 16, dev)[0] == 0
