"""The restatement of a multi-row call (the question chunk and 2..7-row calls), on the CPU.

Row i of a Q-row call over K keys attends, under the causal mask, the n_i = K - Q + i + 1 keys
before it (multibin.py:2210-2218: valid = raw > NEG once the mask is added; tail = valid & ~sel).
The restatement takes the later keys back out of the cluster statistics (oracle.index_downdate)
and runs each row as a decode step at n_i without an index update (oracle.rows_step).

Pins, independent of the GPU code: on integer-valued keys and values every fp32 sum is exact,
so the downdated statistics must equal fresh sums over [0, m) bit for bit, and each row of
rows_step must equal a decode step over a state whose statistics are fresh sums over [0, n_i).
Planted slips (a key taken back at the wrong position, every row run at K) are shown to fail.
"""
import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import D, G, SC, SC2, f32_to_bf16

RNG = np.random.default_rng(2024)
HKV_T = 2
R_T = HKV_T * G


def _sums(Kf, Vf, asg, m, C):
    """nb, Sk, Sk2, Sv of the first m keys per query row (fp64, exact for small integers)."""
    R = asg.shape[0]
    nb = np.zeros((R, C), np.float64)
    Sk = np.zeros((R, C, D), np.float64)
    Sk2 = np.zeros((R, C, D), np.float64)
    Sv = np.zeros((R, C, D), np.float64)
    for r in range(R):
        kv = r // G
        a = asg[r, :m]
        np.add.at(nb[r], a, 1.0)
        np.add.at(Sk[r], a, Kf[kv, :m])
        np.add.at(Sk2[r], a, Kf[kv, :m] ** 2)
        np.add.at(Sv[r], a, Vf[kv, :m])
    return {"nb": nb.astype(np.float32), "Sk": Sk.astype(np.float32), "Sk2": Sk2.astype(np.float32),
            "Sv": Sv.astype(np.float32)}


def _int_state(T, Lmax, C):
    Kf = RNG.integers(-8, 9, (HKV_T, Lmax, D)).astype(np.float32)
    Vf = RNG.integers(-8, 9, (HKV_T, Lmax, D)).astype(np.float32)
    asg = RNG.integers(0, C, (R_T, Lmax)).astype(np.int32)
    st = {"K": f32_to_bf16(Kf), "V": f32_to_bf16(Vf), "asg": asg,
          "codes": RNG.integers(-127, 128, (HKV_T, Lmax, 32)).astype(np.int8),
          "U": RNG.normal(size=(HKV_T, D, 32)).astype(np.float32),
          "scale": RNG.uniform(0.5, 2.0, (HKV_T, 32)).astype(np.float32)}
    st.update(_sums(Kf, Vf, asg, T, C))
    return st, Kf, Vf


def test_index_downdate_equals_fresh_sums_on_exact_data():
    T, Lmax, C = 300, 320, 8
    st, Kf, Vf = _int_state(T, Lmax, C)
    for m in (299, 290, 257):
        s = {k: (v.copy() if k in ("nb", "Sk", "Sk2", "Sv") else v) for k, v in st.items()}
        for p in range(T - 1, m - 1, -1):
            O.index_downdate(s, p, G)
        want = _sums(Kf, Vf, st["asg"], m, C)
        for f in ("nb", "Sk", "Sk2", "Sv"):
            assert np.array_equal(s[f], want[f]), (m, f)
    # a planted slip: the keys taken back one position too high fail the same check
    s = {k: (v.copy() if k in ("nb", "Sk", "Sk2", "Sv") else v) for k, v in st.items()}
    for p in range(T, 290, -1):
        O.index_downdate(s, p, G)
    want = _sums(Kf, Vf, st["asg"], 290, C)
    assert not all(np.array_equal(s[f], want[f]) for f in ("Sk", "Sv"))


@pytest.mark.parametrize("Q", [2, 5, 8])
def test_rows_step_equals_decode_steps_over_fresh_prefix_states(Q):
    """Every row i of rows_step equals a decode step at n_i (no index update) over the same
    index whose statistics are fresh sums over [0, n_i): sel, scores, tail counts, quotas,
    expanded sets and the output, bit for bit."""
    n_keys, Lmax, C, E = 280, 320, 8, 24
    ns, nl, k = 2, 3, 6
    st, Kf, Vf = _int_state(n_keys, Lmax, C)
    q_rows = f32_to_bf16(RNG.normal(size=(Q, R_T, D)).astype(np.float32))
    sm, sm2 = np.float32(SC), np.float32(SC2)
    got = O.rows_step(st, q_rows, n_keys, ns, nl, k, E, G, sm, sm2)
    assert sorted(got) == list(range(Q))
    for i in range(Q):
        n_i = n_keys - Q + i + 1
        fresh = dict(st)
        fresh.update(_sums(Kf, Vf, st["asg"], n_i, C))
        want = O.decode_step(fresh, q_rows[i], n_i, ns, nl, k, E, G, sm, sm2, update_index=False)
        for f in ("sel", "score", "n_t", "quota", "exp_idx", "out"):
            assert np.array_equal(got[i][f], want[f]), (i, f)
        # the row's local window ends at its own position
        assert list(got[i]["sel"][0, ns:ns + nl]) == list(range(n_i - nl, n_i))
    # the input state is left as it was
    assert np.array_equal(st["Sk"], _sums(Kf, Vf, st["asg"], n_keys, C)["Sk"])
    # a planted slip: row 0 run at the call's key count instead of n_0 differs
    wrong = O.decode_step(st, q_rows[0], n_keys, ns, nl, k, E, G, sm, sm2, update_index=False)
    assert not np.array_equal(wrong["sel"], got[0]["sel"])


def test_rows_step_single_row_is_the_decode_step_without_update():
    n_keys, Lmax, C, E = 200, 256, 8, 16
    st, _, _ = _int_state(n_keys, Lmax, C)
    q = f32_to_bf16(RNG.normal(size=(1, R_T, D)).astype(np.float32))
    got = O.rows_step(st, q, n_keys, 1, 2, 5, E, G, np.float32(SC), np.float32(SC2))[0]
    want = O.decode_step(st, q[0], n_keys, 1, 2, 5, E, G, np.float32(SC), np.float32(SC2), update_index=False)
    for f in ("sel", "quota", "exp_idx", "out"):
        assert np.array_equal(got[f], want[f])
