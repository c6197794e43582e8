"""Read-budget accounting of the deployed configurations.

rho = sink + local + top-k + E/N + 1.5 C/N  (run_openattention.sh:16-18; proxies are charged
1.5 KV rows each: mean key, mean value and the diagonal variance).  (C, E) per budget are the
deployed split of run_openattention.sh:27-31 at the accounting context CTX_LEN = 32768
(methods_eager.py:81-84).  At another accounting context (the reference's --ctx-len), C and E
scale with it (run_multibin_hat_bench.py:397-413).

Token counts at a decode step with n keys:
  multibin rule (the accuracy-path oracle, default): sink = local = int(1e-4 * n)
      (SinkMasker / LocalMasker, maskers/base.py:152-158), heavy fraction rounded to 6 digits
      (run_multibin_hat_bench.py:406), k = int(heavy * n)
  deployed rule: sink = local = max(1, int(1e-4 * n)), k = max(1, int(heavy * n))
      (methods_eager.py:605-607).
Both give (3, 3, 9) at n = 32768 and 1%.
"""
from __future__ import annotations

from dataclasses import dataclass

CTX_LEN = 32768
SINK = LOCAL = 0.0001
PROXY_ROWS = 1.5
DEPLOYED = {0.01: (64, 216), 0.03: (192, 679), 0.05: (192, 1335), 0.10: (256, 2877)}


@dataclass(frozen=True)
class Budget:
    rho: float
    C: int
    E: int
    ctx_len: int
    rule: str          # "multibin" | "deployed"

    def heavy_frac(self) -> float:
        h = self.rho - SINK - LOCAL - self.E / self.ctx_len - PROXY_ROWS * self.C / self.ctx_len
        return round(h, 6) if self.rule == "multibin" else h

    def counts(self, n: int) -> tuple[int, int, int]:
        """(ns, nl, k_top) at a decode step with n keys."""
        if self.rule == "multibin":
            ns = nl = int(SINK * n)
            k = int(self.heavy_frac() * n)
        else:
            ns = nl = max(1, int(SINK * n))
            k = max(1, int(self.heavy_frac() * n))
        return ns, nl, k

    def realised_read(self, n: int) -> float:
        ns, nl, k = self.counts(n)
        return (ns + nl + k + self.E + PROXY_ROWS * self.C) / n


def budget(rho: float, ctx_len: int = CTX_LEN, rule: str = "multibin", c_max: int | None = None) -> Budget:
    """The deployed (C, E) split for read fraction rho, scaled to the accounting context.

    c_max caps the cluster count (this build keeps cluster ids as bytes: at most 256); the 1.5
    rows of every proxy a capped split drops go to the exact-read budget E, so rho and the top-k
    share are unchanged."""
    key = round(float(rho), 4)
    if key not in DEPLOYED:
        raise ValueError(f"no deployed (C, E) split for rho={rho}; known: {sorted(DEPLOYED)}")
    if rule not in ("multibin", "deployed"):
        raise ValueError(f"rule must be 'multibin' or 'deployed', got {rule}")
    C0, E0 = DEPLOYED[key]
    if ctx_len == CTX_LEN:
        C, E = C0, E0
    else:
        C = max(1, int(round(C0 * ctx_len / CTX_LEN)))
        E = max(0, int(round(E0 * ctx_len / CTX_LEN)))
    if c_max is not None and C > int(c_max):
        E += int(round(PROXY_ROWS * (C - int(c_max))))
        C = int(c_max)
    b = Budget(rho=float(rho), C=C, E=E, ctx_len=int(ctx_len), rule=rule)
    if b.heavy_frac() <= 0:
        raise ValueError(f"rho={rho} leaves no top-k budget at C={C}, E={E}")
    return b
