"""The per-(device, stream) workspace of the Python wrappers: zero-filled at allocation, reused
while large enough, and grown at least twofold so that a run of growing shapes retires only
logarithmically many buffers (a replaced workspace is kept alive for graphs that captured it)."""

from __future__ import annotations

import pytest
import torch

import _pk

pytestmark = pytest.mark.gpu


def test_workspace_growth_is_geometric(cuda):
    s = torch.cuda.Stream(device=cuda)
    with torch.cuda.stream(s):
        first = _pk.workspace(cuda, 1000)
        assert first.numel() >= 1 << 20 and int(first.sum()) == 0
        assert _pk.workspace(cuda, 5000).data_ptr() == first.data_ptr()  # reused
        retired0 = len(_pk._retired_workspaces)
        sizes = []
        for n in range((1 << 20) + 1, (1 << 20) + 64 * 4096, 4096):  # 64 slightly growing requests
            ws = _pk.workspace(cuda, n)
            assert ws.numel() >= n
            sizes.append(ws.numel())
        grows = len(_pk._retired_workspaces) - retired0
        assert grows == 1, grows  # the first grow doubles past every later request
        assert max(sizes) == 2 * first.numel()
        assert int(_pk.workspace(cuda, 1).sum()) == 0
