"""Helpers for the GPU parity tests: run the fp32 oracle on the same inputs and
measure errors the way the tolerances are stated."""
import numpy as np
import torch

from oracle import gdn
from pseudobrain_amd.workloads import to_numpy

O_TOL = 2e-2   # outputs: infinity-norm relative error vs the fp32 reference
S_TOL = 1e-3   # final states (fp32): infinity-norm relative error


def oracle(q, k, v, g, beta, scale, h0, kernel="chunked", cu_seqlens=None):
    """fp32 oracle on the exact values the GPU sees (bf16 inputs widened exactly)."""
    args = [to_numpy(x).astype(np.float32) for x in (q, k, v, g, beta)]
    h = to_numpy(h0).astype(np.float32)
    if cu_seqlens is not None:
        return gdn.varlen(*args, scale, h, to_numpy(cu_seqlens), kernel)
    return gdn.gated_delta_rule(*args, scale, h, kernel)


def rel_err(x, ref) -> float:
    if isinstance(x, torch.Tensor):
        x = to_numpy(x.float())
    return gdn.rel_inf_error(x, ref)


def report(name, o, o_ref, s=None, s_ref=None):
    eo = rel_err(o, o_ref)
    es = rel_err(s, s_ref) if s is not None else 0.0
    print(f"[{name}] o rel_inf={eo:.3e}  S rel_inf={es:.3e}", flush=True)
    return eo, es


def assert_parity(name, o, o_ref, s=None, s_ref=None, o_tol=O_TOL, s_tol=S_TOL):
    eo, es = report(name, o, o_ref, s, s_ref)
    assert np.isfinite(eo) and eo <= o_tol, f"{name}: output error {eo:.3e} > {o_tol}"
    assert np.isfinite(es) and es <= s_tol, f"{name}: state error {es:.3e} > {s_tol}"


# Lines the full-size oracle checks (varlen and million-token workloads) add for
# the session's closing summary (conftest.pytest_terminal_summary), so their
# per-sequence and per-segment errors show in a quiet run's tail.
SUMMARY: list[str] = []


def summarize(line: str) -> None:
    SUMMARY.append(line)
