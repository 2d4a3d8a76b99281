"""HIP verifier harness: the flow of the reference's ``numerical_correctness.py``
(``verify_op`` over its test plans, ``numerical_correctness.py:257-425, 431-635``)
with libtensor_ops_hip.so as the implementation under test, instead of the CUDA
``verify_*`` programs.  The ground truth is the reference's own ``tensor_ops.c``
(``oracle/_ref/tensor_ops.so``, compiled from the reference source by
``oracle/Makefile``) wherever that library is present, else the restatement
(``oracle/liboracle.so``); ``--against`` picks one explicitly.

For each of the 45 plans (``tests/golden/make_golden.py`` PLANS, the dtype
combinations of ``numerical_correctness.py:432-567``) it draws ``--iterations``
fresh inputs with the plan's generators (``numerical_correctness.py:110-138``,
scale / zero point rules of ``:278-282``), runs the operator through the HIP
library's C ABI on host tensors (the reference's calling convention) and through
the oracle, and checks the parity class of the operator:

* bit-exact for every operator except Gemm / Conv2d / Softmax (NaN results only
  need to be NaN of the format);
* Gemm / Conv2d / Softmax within the tolerance of ``tests/helpers.assert_close``;
  with ``--exact`` (the library's fp64 Gemm / Conv mode) Gemm and Conv2d are
  bit-exact too, Softmax stays in its tolerance class (its exp is evaluated
  with an fp32 core, not glibc's exp).

It prints a per-plan line and the per-operator summary (99th percentile of the
per-iteration max absolute and relative error, as the reference's report does)
and exits non-zero if any iteration falls outside its class.  Test
infrastructure: it needs a GPU and runs only here and in the GPU tests.

    python tests/verify.py [--iterations 20] [--seed 0] [--exact] [--plans 0,5,12]
                           [--against reference|oracle]
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tests.golden.make_golden import PLANS, call, gen  # noqa: E402
from tests.helpers import TOL_OPS, assert_bitexact, assert_close, decode, nan_mask  # noqa: E402


def draw(rng, op, shapes, dts):
    ins = [gen(rng, s, d) if s is not None else None for s, d in zip(shapes, dts)]
    if op in ("quantize_linear", "dequantize_linear"):
        s = np.abs(ins[1].astype(np.float64)) + 1e-4
        ins[1] = s.astype(O.STORAGE[O.NAMES[dts[1]]])
        z = np.round(ins[2].astype(np.float64))
        if op == "quantize_linear":
            z = np.clip(z, -128, 127)
        ins[2] = z.astype(O.STORAGE[O.NAMES[dts[2]]])
    return ins


def errors(got, ref, dt):
    """Max absolute and relative error over the elements where the reference is finite."""
    g, r = decode(got, dt), decode(ref, dt)
    fin = np.isfinite(r) & ~nan_mask(ref, dt)
    if not fin.any():
        return 0.0, 0.0
    d = np.abs(g[fin] - r[fin])
    d = np.where(np.isnan(d), np.inf, d)
    rel = d / np.maximum(np.abs(r[fin]), 1e-30)
    return float(d.max()), float(rel.max())


def tolerance_class(op, exact):
    return op == "softmax" or (op in TOL_OPS and not exact)


def verify(hip, oracle, iterations=20, seed=0, exact=False, plans=None, log=print):
    """Runs the plans; returns (failures, {op: {"abs": [...], "rel": [...]}})."""
    hip.set_exact(exact)
    stats, failures = {}, []
    try:
        for i, (op, shapes, dts, out_dt, params) in enumerate(PLANS):
            if plans is not None and i not in plans:
                continue
            rng = np.random.default_rng([seed, i])
            ok = 0
            st = stats.setdefault(op, {"abs": [], "rel": []})
            for it in range(iterations):
                ins = draw(rng, op, shapes, dts)
                ref = call(oracle, op, ins, dts, out_dt, params)
                what = f"plan{i:02d} {op} {dts}->{out_dt} iter {it}"
                try:
                    got = call(hip, op, ins, dts, out_dt, params)
                    if tolerance_class(op, exact):
                        assert_close(got, ref, out_dt, what=what)
                    else:
                        assert_bitexact(got, ref, out_dt, what=what)
                    ok += 1
                except (AssertionError, RuntimeError) as e:
                    failures.append(str(e)[:400])
                    continue
                a, r = errors(got, ref, out_dt)
                st["abs"].append(a)
                st["rel"].append(r)
            cls = "tolerance" if tolerance_class(op, exact) else "bit-exact"
            log(f"plan{i:02d} {op:<18} {'+'.join(dts):<28} -> {out_dt:<12} {cls:<9} {ok}/{iterations}")
    finally:
        hip.set_exact(False)
    return failures, stats


def summary(stats, log=print):
    log(f"{'operator':<18} | {'abs (99%)':<10} | {'rel (99%)':<10} | samples")
    log("-" * 56)
    for op, st in stats.items():
        if st["abs"]:
            log(f"{op:<18} | {np.percentile(st['abs'], 99):.2e}   | {np.percentile(st['rel'], 99):.2e}   | "
                f"{len(st['abs'])}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--iterations", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--exact", action="store_true", help="fp64 Gemm / Conv mode: Gemm and Conv2d bit-exact as well")
    ap.add_argument("--plans", default=None, help="comma-separated plan indices (default: all)")
    ap.add_argument("--against", choices=("reference", "oracle"), default=None,
                    help="ground truth: the compiled reference tensor_ops.c (default where built) or the "
                         "restatement")
    args = ap.parse_args()
    ref = O.reference()
    against = args.against or ("reference" if ref is not None else "oracle")
    if against == "reference" and ref is None:
        print("verify.py: oracle/_ref/tensor_ops.so is not built (run make -C oracle where the reference "
              "source is present)", file=sys.stderr)
        return 2
    truth = ref if against == "reference" else O.oracle()
    try:
        import torch
        torch.cuda.init()
    except Exception:
        pass
    from tests.helpers import HipLib
    hip = HipLib()
    if hip.device_count() == 0:
        print("verify.py: libtensor_ops_hip.so reports no GPU", file=sys.stderr)
        return 2
    plans = {int(p) for p in args.plans.split(",")} if args.plans else None
    print(f"ground truth: {against} ({truth.path})")
    failures, stats = verify(hip, truth, args.iterations, args.seed, args.exact, plans)
    print()
    summary(stats)
    for f in failures[:20]:
        print("FAIL", f)
    print(f"{len(failures)} failing iterations")
    return 1 if failures else 0


if __name__ == "__main__":
    sys.exit(main())
