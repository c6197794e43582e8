"""oa_flash_decode_noalloc (split partials in the library's fixed device array, nothing
allocated) against oa_flash_decode with caller workspaces, through the C ABI: bit-exact on two
calls in a row, the second with a smaller input, so stale contents of the shared array from the
first call cannot leak into the second."""
import math

import numpy as np
import pytest
import torch

from openattention_amd import lib, ops
from tests.helpers import D, HKV, HQ, SC

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(seed, B, Lmax, Cn, Ns, Ne, pads):
    g = torch.Generator().manual_seed(seed)
    R, BH = B * HQ, B * HKV
    k = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16)
    v = torch.randn(BH, Lmax, D, generator=g).to(torch.bfloat16)
    q = torch.randn(R, D, generator=g).to(torch.bfloat16)
    perm = torch.stack([torch.randperm(Lmax, generator=g) for _ in range(R)])
    sel, ex = perm[:, :Ns].int(), perm[:, Ns:Ns + Ne].int().clone()
    ex[:, Ne - pads:] = -1
    kb = torch.randn(R, Cn, D, generator=g).to(torch.bfloat16)
    vb = torch.randn(R, Cn, D, generator=g).to(torch.bfloat16)
    ln = torch.rand(R, Cn, generator=g) * 5
    ln[:, :3] = -math.inf
    ex[1, :] = -1
    sel[1, :] = -1
    ln[1, :] = -math.inf                     # row 1: nothing valid -> 0
    return [t.to(DEV) for t in (q, k, v, sel, ex, kb, vb, ln)]


@pytest.mark.parametrize("first,second", [
    # (seed, B, Lmax, C, Ns, Ne, pads, n_split): the second call is smaller in rows, split and list
    ((11, 2, 2048, 64, 15, 216, 9, 8), (12, 1, 1024, 16, 7, 40, 3, 3)),
    ((13, 1, 4096, 64, 15, 216, 0, 16), (14, 1, 4096, 64, 15, 100, 20, 2)),
])
def test_flash_noalloc_equals_workspace_entry(first, second):
    for seed, B, Lmax, Cn, Ns, Ne, pads, n_split in (first, second):
        print(f"[case] flash noalloc seed={seed} B={B} C={Cn} Ns={Ns} Ne={Ne} split={n_split}", flush=True)
        q, k, v, sel, ex, kb, vb, ln = _case(seed, B, Lmax, Cn, Ns, Ne, pads)
        ref = ops.flash_decode(q, k, v, sel, ex, kb, vb, ln, proxy_per_kv=False, sm_scale=SC,
                               n_split=n_split)
        out = torch.full_like(q, float("nan"))
        got = ops.flash_decode(q, k, v, sel, ex, kb, vb, ln, proxy_per_kv=False, sm_scale=SC,
                               n_split=n_split, out=out, noalloc=True)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        a = got.view(torch.int16).cpu().numpy()
        b = ref.view(torch.int16).cpu().numpy()
        assert np.array_equal(a, b), f"noalloc differs from the workspace entry in {np.sum(a != b)} values"
        assert np.all(got[1].float().cpu().numpy() == 0)


def test_flash_noalloc_rejects_oversized_split():
    """rows * n_split * 130 above the 4 MiB array is refused before any launch."""
    q, k, v, sel, ex, kb, vb, ln = _case(15, 1, 1024, 8, 4, 8, 0)
    out = torch.empty_like(q)
    with pytest.raises(RuntimeError, match="status -28"):
        ops.flash_decode(q, k, v, sel, ex, kb, vb, ln, proxy_per_kv=False, sm_scale=SC,
                         n_split=256, out=out, noalloc=True)       # 32 * 256 * 130 > 2^20
    # the library still works afterwards
    ok = ops.flash_decode(q, k, v, sel, ex, kb, vb, ln, proxy_per_kv=False, sm_scale=SC,
                          n_split=4, out=out, noalloc=True)
    ref = ops.flash_decode(q, k, v, sel, ex, kb, vb, ln, proxy_per_kv=False, sm_scale=SC, n_split=4)
    torch.cuda.synchronize()
    assert torch.equal(ok.view(torch.int16), ref.view(torch.int16))
    assert lib.load().oa_abi_version() >= 1
