"""The static query metric loader (the reference's packed upper-triangular asset format)."""
import os

import pytest
import torch

from openattention_amd import synth
from openattention_amd.static_metric import load_static_metric, pack_triu, unpack_triu

REF_ASSET = "/root/reference/assets/llama-3.1-8b-instruct.query_metric.triu.pt"


def test_pack_unpack_roundtrip(tmp_path):
    st = synth.static_metric(2)
    M = st["M"]
    packed = {"M_triu": pack_triu(M), "dim": 128, "inv_freq": st["inv_freq"], "attention_scaling": 1.0,
              "space": "pre-rope", "source": "synthetic", "n_requests": 0}
    path = str(tmp_path / "m.triu.pt")
    torch.save(packed, path)
    got = load_static_metric(path)
    assert torch.equal(got["M"], M)
    assert torch.equal(got["inv_freq"], st["inv_freq"].float())
    assert got["attention_scaling"] == 1.0 and got["source"] == "synthetic"


def test_rejects_malformed(tmp_path):
    path = str(tmp_path / "bad.pt")
    torch.save({"M_triu": torch.zeros(2, 2, 10), "dim": 128, "inv_freq": torch.zeros(64)}, path)
    with pytest.raises(ValueError):
        load_static_metric(path)
    torch.save({"weights": torch.zeros(3)}, path)
    with pytest.raises(ValueError):
        load_static_metric(path)
    with pytest.raises(ValueError):
        unpack_triu(torch.zeros(5), 3)


@pytest.mark.skipif(not os.path.exists(REF_ASSET), reason="reference checkout not present")
def test_reference_asset():
    """The asset the reference ships (32 layers x 32 query heads): symmetric positive
    semi-definite metrics, Llama-3.1 RoPE frequencies (rope_theta 500000 with the 8x
    low-frequency scaling: the highest frequency is 1, the lowest below the unscaled one)."""
    st = load_static_metric(REF_ASSET)
    M = st["M"]
    assert M.shape == (32, 32, 128, 128)
    assert torch.equal(M, M.transpose(-1, -2))
    ev = torch.linalg.eigvalsh(M[::8, ::8].double())
    assert float(ev.min()) > -1e-6 * float(ev.max())
    inv = st["inv_freq"]
    assert inv.shape == (64,) and float(inv[0]) == 1.0
    assert torch.all(inv[1:] < inv[:-1])
    assert float(inv[-1]) < 500000.0 ** (-126 / 128)
