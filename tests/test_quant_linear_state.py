"""QuantLinear's state dict keeps pack_int4_n order whatever the layout in memory, and loading
never rewrites the caller's tensors: with ``load_state_dict(..., assign=True)`` torch hands the
caller's own tensor to the module, which must not be converted to blocks in place (a second
load of the same dict would otherwise convert it twice). CPU only: no kernel runs."""

from __future__ import annotations

import torch

import quant_linear as ql


def _layer() -> ql.QuantLinear:
    q = ql.QuantLinear(256, 512, bias=True, group_size=128)
    assert q.tiled
    g = torch.Generator().manual_seed(3)
    words = torch.randint(-2**31, 2**31 - 1, (256, 64), generator=g, dtype=torch.int64).to(torch.int32)
    q.set_codes(words)
    q.scales.copy_(torch.rand(2, 512, generator=g).half())
    q.bias.copy_(torch.randn(512, generator=g).half())
    return q


def test_state_dict_round_trip_and_assign_twice():
    src = _layer()
    sd = src.state_dict()
    codes = src.codes().clone()
    assert torch.equal(sd["qweight"], codes)          # pack_int4_n order in the dict
    snapshot = {k: v.clone() for k, v in sd.items()}
    for assign in (False, True, True):
        dst = ql.QuantLinear(256, 512, bias=True, group_size=128)
        dst.load_state_dict(sd, assign=assign)
        assert torch.equal(dst.codes(), codes)
        assert torch.equal(dst.qweight, src.qweight)  # blocks in memory
        for k, v in sd.items():                       # the caller's dict is untouched
            assert torch.equal(v, snapshot[k]), k
