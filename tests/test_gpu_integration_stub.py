"""The ctypes stub of the integration guide (section 3), run as written.

The guide shows how a maintainer would bind `lkv_select_decode` inside the reference: its own
ctypes structures, argument types and call, replacing `rank` + `gather_zerocopy` + `attend` for
one selecting layer. This test executes that code block from the guide itself on a layer laid out
as the reference's `TieredLayer` holds it (the host pool's device alias, the two GPU slots of sink
and current, the metadata), and holds it to the library's own binding (bit for bit: the same
entry point) and to the float64 oracle over the selected set (within 2e-3, plus the bfloat16
output's rounding).
"""

from __future__ import annotations

import os
import re
from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _stub() -> dict:
    text = (ROOT / "INTEGRATION.md").read_text()
    block = re.search(r"## 3\. The C ABI directly.*?```python\n(.*?)```", text, re.S).group(1)
    ns: dict = {}
    cwd = os.getcwd()
    os.chdir(ROOT)  # the stub loads the library by its path from the repository root
    try:
        exec(compile(block, "INTEGRATION.md, section 3", "exec"), ns)
    finally:
        os.chdir(cwd)
    return ns


class _ReferenceLayout:
    """What the stub reads from a reference TieredLayer (lazykv/tiered.py:243-302): `host_dev`, the
    device alias of the bf16 host pool [cap, h, 2, bs, d]; `pool`, the GPU slots [2, h, 2, bs, d]
    (sink, current); `kmin` / `kmax` [1, h, cap, d]; `block_size`, `k_blocks`."""

    def __init__(self, h: int, g: int, n: int, bs: int, d: int, k: int) -> None:
        from lazykv_amd import kernels
        from lazykv_amd.pinned import device_view, pinned_empty
        from lazykv_amd.workload import draw_layer, to_pool

        w = draw_layer(0, h * g, h, d, n * bs, bs, torch.bfloat16, device="cuda")
        self.query = w.query.contiguous()
        full = to_pool(w.keys, w.values, bs)
        self.host = pinned_empty(tuple(full.shape), torch.bfloat16)
        self.host.copy_(full)
        self.host_dev = device_view(self.host)
        self.pool = full[[0, n - 1]].contiguous()
        self.kmin = torch.zeros((1, h, n, d), dtype=torch.bfloat16, device="cuda")
        self.kmax = torch.zeros_like(self.kmin)
        kernels.store_blocks(kernels.dense_source(w.keys, w.values, bs), n_kv=h, head_dim=d, block_size=bs, first_block=0, n_blocks=n - 1,
                             kmin=self.kmin, kmax=self.kmax)
        self.full = full
        self.block_size, self.k_blocks = bs, k


@pytest.mark.parametrize(("h", "g", "n", "d", "k"), [(8, 4, 300, 128, 32), (2, 8, 120, 128, 17)])
def test_the_guides_ctypes_stub_is_the_select_decode_call(h: int, g: int, n: int, d: int, k: int) -> None:
    from lazykv_amd import kernels
    from oracle import reference as R

    ns = _stub()
    layer = _ReferenceLayout(h, g, n, 16, d, k)
    n_sealed, fill, scale = n - 1, 16, d**-0.5
    out, lse = ns["decode_layer"](layer, layer.query.view(1, h * g, 1, d), scale, n_sealed, fill)
    ids = torch.empty((h, k), dtype=torch.int32, device="cuda")
    ss = kernels.pool_source(layer.pool)
    want_o, want_l = kernels.select_decode(layer.query, layer.kmin, layer.kmax, k, cand_offset=1, n_cand=n_sealed - 1, block_size=16, scale=scale,
                                           sel=kernels.pool_source(layer.host), sink=ss, sink_block=0, cur=ss, cur_block=1, fill=fill, out_idx=ids)
    torch.cuda.synchronize()
    assert torch.equal(out.view(h * g, d), want_o) and torch.equal(lse, want_l)
    # The oracle over sink + the selected blocks + the current block's first `fill` tokens.
    pool = layer.full.double().cpu().numpy()

    def bkv(j: int, b: int):  # noqa: ANN202
        return pool[b, j, 0], pool[b, j, 1]

    ks, vs = R.gathered_tokens(bkv, h, ids.cpu().numpy(), 0, n_sealed, fill, 16)
    o64, l64 = R.attend_tokens(layer.query.double().cpu().numpy(), ks, vs, scale)
    # The stub writes bfloat16: within 2e-3 of the truth plus the output's own rounding (2^-8 of |out|).
    assert (np.abs(out.view(h * g, d).float().cpu().numpy() - o64) <= 2e-3 + 2.0**-8 * np.abs(o64)).all()
    assert np.abs(lse.cpu().numpy() - l64).max() < 2e-3
