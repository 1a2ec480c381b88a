"""Definition runner: the MI355X counterpart of the reference harness for quant_gemm definitions.

The reference tests one kernel per definition JSON with UnifiedTestRunner
(kernelevalplus-main/llm_kernel_test/unified_test_runner.py:129-204) and QuantGEMMHandler
(op_test_handler.py:128-458): compile the attempt's kernel.cu, generate inputs
(torch.randn weights quantised by quantize_to_q4_0 / q4_1 / q8_0, randn fp32
activations), gate correctness by NMSE against dequantise-then-fp32-matmul, time 100
calls after 10 warm-up calls, compare the first configuration with the GGML baseline,
and write test_results.json.  This module does the same for libksq:

  compilation  load libksq.so and resolve the definition's entry point (no JIT)
  correctness  the harness NMSE gate (threshold from the definition, default 0.05,
               plus no NaN / Inf), and the exact checks of this path on sampled rows and
               columns: activation quantisation bit-exact, integer block dots bit-exact,
               fp32 outputs within 1e-3 of the fp64 block formula (ksq.refcheck)
  performance  the harness timing (10 warm-up + 100 eager forward calls between two
               events: latency_ms_eager) and the device time of the same call replayed
               from a HIP graph (latency_ms, which tflops / gflops / gbps use); inputs
               stay cache-resident as in the reference
  baseline     every configuration against the GGML table the reference compares with
               (data/ggml_baseline_quant_gemm.json), for one chosen hardware

    python -m ksq.runner --definition path/to/def.json [--attempt-path DIR]
    python -m ksq.runner --definition path/to/variants/<model>/<variant> [--attempt-path DIR]
    python -m ksq.runner --operators path/to/core/operators [--attempt-path DIR]
    python -m ksq.runner --sweep [--filter TEXT] [--all-configs] [--out results.json]

--all-configs uses the definition's own test_configs (M = 1, 2, 3, 4, 5, 8, 512) instead
of the handler's three (M = 1, 8, 512; op_test_handler.py:445-453, which the reference
runner uses whenever they exist).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
import zlib
from datetime import datetime

import numpy as np
import torch

from . import _lib, ops, refcheck

DATA = os.path.join(os.path.dirname(os.path.abspath(__file__)), "data")

# weight dtype of a definition -> (weight type code, entry point of include/ksq.h)
WEIGHT_ENTRIES = {
    "q4_0": (_lib.W_Q4_0, "gemm_w4a32c8_q4_0_fp32_int8"),
    "q8_0": (_lib.W_Q8_0, "gemm_w8a32c8_q8_0_fp32_int8"),
    "q4_1": (_lib.W_Q4_1, "gemm_w4a32c8_q4_1_fp32_int8"),
    "q5_0": (_lib.W_Q5_0, "gemm_w5a32c8_q5_0_fp32_int8"),
    "q5_1": (_lib.W_Q5_1, "gemm_w5a32c8_q5_1_fp32_int8"),
}
# activation types of the fp32-input entries, and the device / numpy quantiser of each
FP32_ACTIVATIONS = (_lib.A_F32, _lib.A_F32_Q8S, _lib.A_F32_Q8F_RNE, _lib.A_F32_Q8F_LROUND)
BLOCK_BYTES = {_lib.W_Q4_0: 18, _lib.W_Q8_0: 34, _lib.W_Q4_1: 20, _lib.W_Q5_0: 22, _lib.W_Q5_1: 24}
HANDLER_CONFIGS = ((1, "single_token"), (8, "small_batch"), (512, "large_batch"))


# ---------------------------------------------------------------- spec handling
def load_spec(path: str) -> dict:
    """A definition JSON, an operator spec.json, or an operator variant directory (its spec.json
    plus impl.json) as the runner's spec dict.  For spec.json files the variant directory and
    its impl.json are recorded too (core/operators/registry.py:97-136 reads a variant's spec.json
    from its directory; impl.json carries the kernel's file and entry point)."""
    vdir = None
    if os.path.isdir(path):
        vdir, path = path, os.path.join(path, "spec.json")
    with open(path) as f:
        spec = json.load(f)
    if vdir is None and os.path.basename(path) == "spec.json":
        vdir = os.path.dirname(os.path.abspath(path))
    if vdir is not None:
        spec["_variant_dir"] = os.path.abspath(vdir)
        ipath = os.path.join(vdir, "impl.json")
        if os.path.exists(ipath):
            with open(ipath) as f:
                impl = json.load(f)
            spec["_impl"] = impl
            if "kernel" not in spec and isinstance(impl.get("kernel"), dict):
                spec["kernel"] = impl["kernel"]
    if "params" not in spec and "axes" in spec:   # unified_test_runner.py:111-126
        spec["params"] = {k: ({"value": v.get("value")} if v.get("type") == "const" else {"default": 1})
                          for k, v in spec["axes"].items() if isinstance(v, dict)}
    return spec


def discover(operators_dir: str, family: str = "quant_gemm") -> list[dict]:
    """Every variant of an operator family, as the reference's OperatorRegistry finds them
    (core/operators/registry.py:71-136: <family>/manifest.json, then variants/<variant>/spec.json),
    also one level further down (variants/<model>/<variant>/spec.json, where the reference keeps
    its deepseek_v2 and deepseek_v3 operators).  Each entry is a loaded spec (load_spec) with its
    variant path relative to variants/ in "_variant"."""
    fdir = os.path.join(operators_dir, family)
    if not os.path.exists(os.path.join(fdir, "manifest.json")):
        raise FileNotFoundError(f"{fdir}: no manifest.json (not an operator family directory)")
    vroot = os.path.join(fdir, "variants")
    found = []
    for root, dirs, files in os.walk(vroot):
        dirs.sort()
        if "spec.json" in files:
            spec = load_spec(root)
            spec["_variant"] = os.path.relpath(root, vroot)
            found.append(spec)
    return found


def _arch_tags(spec: dict) -> list[str]:
    """Model-architecture qualifiers of a spec: its model_architectures ("deepseek-v2" ->
    "deepseek_v2") and the model directory its variant sits under (variants/deepseek_v2/...)."""
    tags = [a.lower().replace("-", "_").replace(".", "_") for a in spec.get("model_architectures") or []]
    rel = spec.get("_variant")
    if rel is None and spec.get("_variant_dir"):
        parts = os.path.normpath(spec["_variant_dir"]).split(os.sep)
        if "variants" in parts:
            rel = os.sep.join(parts[parts.index("variants") + 1:])
    if rel:
        parts = os.path.normpath(rel).split(os.sep)
        if len(parts) > 1:
            tags.append(parts[0].lower().replace("-", "_"))
    return list(dict.fromkeys(tags))


def spec_from_table(d: dict) -> dict:
    """A spec from one entry of data/quant_gemm_definitions.json."""
    return {
        "name": d["name"], "op_type": "quant_gemm",
        "axes": {"M": {"type": "var"}, "N": {"type": "const", "value": d["N"]},
                 "K": {"type": "const", "value": d["K"]}},
        "inputs": {"weight": {"dtype": d["weight_dtype"]}, "activation": {"dtype": d["activation_dtype"]}},
        "test_configs": [{"name": f"batch_{m}", "M": m, "N": d["N"], "K": d["K"]} for m in d["M"]],
        "accuracy": {"threshold": d["threshold"]} if d.get("threshold") is not None else None,
    }


def _dim(spec: dict, cfg: dict, name: str, default: int) -> int:
    if name in cfg:
        return int(cfg[name])
    ax = spec.get("axes", {}).get(name)
    if isinstance(ax, dict):
        return int(ax.get("value", ax.get("default", default)) if ax.get("type") == "const"
                   else ax.get("default", default))
    p = spec.get("params", {}).get(name, {})
    return int(p.get("value", p.get("default", default))) if isinstance(p, dict) else default


def entry_candidates(spec: dict) -> list[str]:
    """libksq symbols that may implement a spec, in the order they are tried.  First the
    variant-qualified names gemm_{name}_{arch} for the spec's model architectures (a variant
    whose arithmetic differs from the generic operator of the same name, such as the deepseek_v2
    W4A32C8 operator with its fp32 activation scales, is exported under that name); then the
    reference's own order (core/run_tests.py:218-234): kernel.entry_point, gemm_{name}, name."""
    name = spec.get("name", "")
    entry = (spec.get("kernel") or {}).get("entry_point") or name
    out = []
    for tag in _arch_tags(spec):
        out += [f"gemm_{name}_{tag}", f"{entry}_{tag}"]
    out += [entry, f"gemm_{name}", name]
    return list(dict.fromkeys(c for c in out if c))


def resolve(spec: dict) -> tuple[int, int, str]:
    """(weight type, activation type, entry point) for a spec: the first entry_candidates() name
    that libksq implements, else (definition JSONs, whose names are shapes) the entry of the
    weight dtype."""
    wd = spec["inputs"]["weight"]["dtype"].replace("block_", "")
    ad = spec["inputs"]["activation"]["dtype"]
    if ad not in ("float32", "fp32"):
        raise ValueError(f"activation dtype {ad!r}: only fp32-activation definitions are defined for quant_gemm")
    for c in entry_candidates(spec):
        if c in ops.ENTRY_POINTS and ops.ENTRY_POINTS[c][1] in FP32_ACTIVATIONS:
            wt, at = ops.ENTRY_POINTS[c]
            if WEIGHT_ENTRIES.get(wd, (wt,))[0] != wt:
                raise ValueError(f"entry {c} takes weight type {wt}, the spec's weight is {wd!r}")
            return wt, at, c
    if wd not in WEIGHT_ENTRIES:
        raise ValueError(f"weight dtype {wd!r} has no libksq entry")
    wt, e = WEIGHT_ENTRIES[wd]
    return wt, _lib.A_F32, e


def test_configs(spec: dict, all_configs: bool) -> list[dict]:
    N, K = _dim(spec, {}, "N", 4096), _dim(spec, {}, "K", 4096)
    if all_configs and spec.get("test_configs"):
        return [{"name": c.get("name", f"M{c.get('M', 1)}"), "M": int(c.get("M", 1)),
                 "N": int(c.get("N", N)), "K": int(c.get("K", K))} for c in spec["test_configs"]]
    return [{"name": n, "M": m, "N": N, "K": K} for m, n in HANDLER_CONFIGS]


# ---------------------------------------------------------------- inputs (op_test_handler.py:174-223)
def _f16_bytes(v: torch.Tensor) -> torch.Tensor:
    return v.to(torch.float16).contiguous().view(torch.uint8).reshape(*v.shape, 2)


def quantize_weights(wf: torch.Tensor, wtype: int) -> torch.Tensor:
    """fp32 [N, K] -> [N, K/32, bytes] with the harness quantisers (llm_kernel_test/reference/
    quantize.py: quantize_to_q8_0 :12-53, quantize_to_q4_0 :56-103, quantize_to_q4_1 :105-153;
    round half to even), computed on the device.  Q5_0 / Q5_1, which the harness cannot
    generate, use the published GGML quantisers (d = v / -16 for the element v of largest
    magnitude; d = (max - min) / 31, m = min)."""
    N, K = wf.shape
    xb = wf.reshape(N, K // 32, 32)
    if wtype == _lib.W_Q8_0:
        amax = xb.abs().amax(-1)
        sc = torch.where(amax > 0, amax / 127.0, torch.ones_like(amax))
        q = torch.round(xb / sc[..., None]).clamp(-128, 127).to(torch.int8)
        return torch.cat([_f16_bytes(sc), q.view(torch.uint8)], -1).contiguous()
    if wtype in (_lib.W_Q4_0, _lib.W_Q4_1):
        if wtype == _lib.W_Q4_0:
            amax = xb.abs().amax(-1)
            sc = torch.where(amax > 0, amax / 7.0, torch.ones_like(amax))
            q = torch.round(xb / sc[..., None] + 8.0).clamp(0, 15).to(torch.uint8)
            head = _f16_bytes(sc)
        else:
            lo, hi = xb.amin(-1), xb.amax(-1)
            sc = torch.where(hi > lo, (hi - lo) / 15.0, torch.ones_like(lo))
            q = torch.round((xb - lo[..., None]) / sc[..., None]).clamp(0, 15).to(torch.uint8)
            head = torch.cat([_f16_bytes(sc), _f16_bytes(lo)], -1)
        return torch.cat([head, q[..., :16] | (q[..., 16:] << 4)], -1).contiguous()
    # Q5_0 / Q5_1
    if wtype == _lib.W_Q5_0:
        idx = xb.abs().argmax(-1, keepdim=True)
        vmax = torch.gather(xb, -1, idx)[..., 0]
        d = vmax / -16.0
        inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
        q = torch.clamp(torch.trunc(xb * inv[..., None] + 16.5), 0, 31).to(torch.int32)
        head = _f16_bytes(d)
    else:
        lo, hi = xb.amin(-1), xb.amax(-1)
        d = (hi - lo) / 31.0
        inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
        q = torch.clamp(torch.trunc((xb - lo[..., None]) * inv[..., None] + 0.5), 0, 31).to(torch.int32)
        head = torch.cat([_f16_bytes(d), _f16_bytes(lo)], -1)
    bit = (q >> 4) & 1
    qh = (bit << torch.arange(32, device=wf.device, dtype=torch.int32)).sum(-1).to(torch.int32)
    qh_bytes = torch.stack([(qh >> (8 * i)) & 0xFF for i in range(4)], -1).to(torch.uint8)
    qs = ((q[..., :16] & 15) | ((q[..., 16:] & 15) << 4)).to(torch.uint8)
    return torch.cat([head, qh_bytes, qs], -1).contiguous()


def dequantize_weights(w: torch.Tensor, wtype: int) -> torch.Tensor:
    """[N, nb, bytes] -> fp32 [N, K] on the device (the dequantisation of gemm_ref.py)."""
    N, nb, _ = w.shape
    lay = refcheck.LAYOUT[wtype]
    d = w[..., 0:2].contiguous().view(torch.float16)[..., 0].float()
    if lay[5] == "i8":
        q = w[..., 2:34].contiguous().view(torch.int8).float()
        return (d[..., None] * q).reshape(N, nb * 32)
    qs = w[..., lay[4]:lay[4] + 16].to(torch.int32)
    q = torch.cat([qs & 15, qs >> 4], -1)
    if lay[5] == "nib5":
        hb = w[..., lay[3]:lay[3] + 4].to(torch.int32)
        h = hb[..., 0] | (hb[..., 1] << 8) | (hb[..., 2] << 16) | (hb[..., 3] << 24)
        q = q + 16 * ((h[..., None] >> torch.arange(32, device=w.device, dtype=torch.int32)) & 1)
    q = q.float()
    if wtype == _lib.W_Q4_0:
        v = d[..., None] * (q - 8.0)
    elif wtype == _lib.W_Q5_0:
        v = d[..., None] * (q - 16.0)
    else:
        m = w[..., 2:4].contiguous().view(torch.float16)[..., 0].float()
        v = d[..., None] * q + m[..., None]
    return v.reshape(N, nb * 32)


# ---------------------------------------------------------------- baseline table
_BASELINE = None


def ggml_baseline(wtype: int, N: int, M: int, K: int, hardware: str):
    """GGML [tflops, us_per_run] for the case, or None (core/tools/baseline_api.py key form)."""
    global _BASELINE
    if _BASELINE is None:
        with open(os.path.join(DATA, "ggml_baseline_quant_gemm.json")) as f:
            _BASELINE = json.load(f)["cases"]
    t = {v[0]: k for k, v in WEIGHT_ENTRIES.items()}.get(wtype)
    if t is None:
        return None
    key = f"w{'4' if t.startswith('q4') else '8'}a32c8_{t}_f32_m{N}_n{M}_k{K}"
    return (_BASELINE.get(key) or {}).get(hardware)


def _quantisers(atype: int):
    """(device quantiser, numpy quantiser) of the activation blocks an fp32 entry of type atype
    forms: block_q8_1, block_q8s (the native W8A8C8 operator) or block_q8f (deepseek_v2 / lm_head)."""
    if atype == _lib.A_F32_Q8S:
        return ops.quantize_q8s, refcheck.quantize_q8s
    if atype in (_lib.A_F32_Q8F_RNE, _lib.A_F32_Q8F_LROUND):
        rule = _lib.Q8F_RNE if atype == _lib.A_F32_Q8F_RNE else _lib.Q8F_LROUND
        return (lambda x: ops.quantize_q8f(x, rule)), (lambda x: refcheck.quantize_q8f(x, rule))
    return ops.quantize_q8_1, refcheck.quantize_q8_1


# ---------------------------------------------------------------- one definition
class DefinitionRunner:
    def __init__(self, warmup: int = 10, iterations: int = 100, baseline_hardware: str = "RTX4090",
                 all_configs: bool = False, seed: int = 0, log=print):
        self.warmup, self.iterations = warmup, iterations
        self.hardware, self.all_configs, self.seed = baseline_hardware, all_configs, seed
        self.log = log
        self.dev = torch.device("cuda:0")

    def run(self, spec: dict, attempt_dir: str | None = None) -> dict:
        name = spec.get("name", "definition")
        res = {"attempt_id": name, "variant": "libksq", "op_type": "quant_gemm",
               "tested_at": datetime.now().isoformat(),
               "spec": {k: v for k, v in spec.items() if not k.startswith("_")},
               "compilation": {}, "correctness": {}, "performance": {}}
        try:
            wtype, atype, entry = resolve(spec)
            getattr(_lib.lib(), entry)
            res["compilation"] = {"success": True, "errors": [], "warnings": [], "diagnostics": [],
                                  "library": _lib.LIB_PATH, "entry_point": entry,
                                  "candidates": entry_candidates(spec), "weight_type": wtype,
                                  "activation_type": atype}
            if spec.get("_variant_dir"):
                res["variant_dir"] = spec["_variant_dir"]
        except Exception as e:  # noqa: BLE001 - reported in the results like a compile error
            res["compilation"] = {"success": False, "errors": [str(e)], "warnings": [], "diagnostics": []}
            return self._save(res, attempt_dir)
        cfgs = test_configs(spec, self.all_configs)
        threshold = (spec.get("accuracy") or {}).get("threshold")
        threshold = 0.05 if threshold is None else threshold   # unified_test_runner.py:410
        N, K = cfgs[0]["N"], cfgs[0]["K"]
        g = torch.Generator(device=self.dev)
        g.manual_seed(self.seed + zlib.crc32(name.encode()))
        wf = torch.randn((N, K), generator=g, device=self.dev, dtype=torch.float32)
        w = quantize_weights(wf, wtype)
        del wf
        wdq = dequantize_weights(w, wtype)
        cases, benches, all_ok, nmses = [], [], True, []
        for c in cfgs:
            M = c["M"]
            x = torch.randn((M, K), generator=g, device=self.dev, dtype=torch.float32)
            case = self._correctness(w, wdq, x, wtype, atype, entry, M, N, K, threshold, g)
            case["config"] = c["name"]
            cases.append(case)
            nmses.append(case["nmse"])
            all_ok &= case["passed"]
            self.log(f"  {name} {c['name']} (M={M}): {'PASS' if case['passed'] else 'FAIL'} nmse={case['nmse']:.2e}"
                     f" exact={case['exact']['passed']}")
            if case["passed"]:
                b = self._performance(w, x, entry, M, N, K, wtype)
                b["config"] = c["name"]
                benches.append(b)
                self.log(f"  {name} {c['name']}: {b['latency_ms'] * 1e3:.2f} us, {b['tflops']} TFLOPS, "
                         f"{b['gbps']} GB/s" + (f", {b['vs_ggml_pct']}% of GGML {self.hardware}"
                                               if b.get("vs_ggml_pct") is not None else ""))
            del x
        res["correctness"] = {"passed": all_ok, "test_cases": cases, "nmse": round(float(np.mean(nmses)), 8),
                              "threshold": threshold}
        res["performance"] = {"benchmarks": benches, "timing": "latency_ms: HIP-graph replay of the call "
                              "(device time); latency_ms_eager: the reference's 100-call event loop",
                              "baseline_comparison": self._first_comparison(benches, wtype, cfgs, N, K)}
        del w, wdq
        return self._save(res, attempt_dir)

    def _correctness(self, w, wdq, x, wtype, atype, entry, M, N, K, threshold, g) -> dict:
        y = ops.forward(w, x, M, N, K, entry=entry)
        ref = x @ wdq.t()                                    # harness reference: dequantise, fp32 matmul
        torch.cuda.synchronize()
        nmse = (torch.mean((y - ref) ** 2) / (torch.mean(ref ** 2) + 1e-10)).item()
        finite = bool(torch.isfinite(y).all().item())
        exact = self._exact(w, x, y, wtype, atype, M, N, K, g)
        return {"passed": bool(nmse <= threshold and finite and exact["passed"]), "nmse": round(nmse, 8),
                "finite": finite, "exact": exact}

    def _exact(self, w, x, y, wtype, atype, M, N, K, g) -> dict:
        """Sampled rows x columns of the definition's own call: quantised activations bit-exact,
        fp32 within 1e-3 of the fp64 block formula.  Then the same entry on unit-scale inputs
        (refcheck "unit-scale exactness"): its outputs must equal the exact integer sums of the
        block dots, which checks the integer block dots of the engine that produced them."""
        rows = sorted({0, M - 1, *torch.randint(0, M, (2,), generator=g, device=self.dev).tolist()})
        cols = sorted(set(torch.randint(0, N, (64,), generator=g, device=self.dev).tolist()) | {0, N - 1})
        xr = x[rows].contiguous()
        dev_q, np_q = _quantisers(atype)
        a_dev = dev_q(xr)
        torch.cuda.synchronize()
        x_np, w_np = xr.cpu().numpy(), w[cols].contiguous().cpu().numpy()
        a_ref = np_q(x_np)
        q_ok = bool(np.array_equal(a_dev.cpu().numpy(), a_ref))
        if atype == _lib.A_F32_Q8S:
            ref64 = refcheck.gemm_q8s_f64(a_ref, w_np)
        elif atype in (_lib.A_F32_Q8F_RNE, _lib.A_F32_Q8F_LROUND):
            ref64, _ = refcheck.exact_gemm(wtype, a_ref, w_np)   # block_q8f: fp32 d_a and s_a
        else:
            ref64 = refcheck.gemm_f64(wtype, a_ref, w_np)
        err = refcheck.max_rel_err(y[rows][:, cols].cpu().numpy(), ref64)
        s_ok, engines = self._unit_scale(wtype, atype, M, N, K, cols)
        return {"passed": q_ok and s_ok and err <= 1e-3, "quantize_bit_exact": q_ok, "block_dots_bit_exact": s_ok,
                "max_rel_err_vs_fp64": err, "rows": rows, "columns_sampled": len(cols), "engines": engines}

    def _unit_scale(self, wtype, atype, M, N, K, cols):
        rng = np.random.default_rng(self.seed + 17 * M + N)
        wu = refcheck.unit_weights(wtype, rng, N, K)
        xu = refcheck.unit_activations(rng, M, K, qmax=refcheck.unit_qmax(wtype, K),
                                       onehot=refcheck.onehot_pattern(M, K // 32))
        q8s = atype == _lib.A_F32_Q8S
        yu = ops.gemm(wtype, atype, torch.from_numpy(wu).to(self.dev), torch.from_numpy(xu).to(self.dev), M, N, K)
        engines = sorted(ops.last_engines())
        au = _quantisers(atype)[1](xu)
        ref, bound = refcheck.exact_gemm(wtype, au, wu[cols], q8s=q8s)
        ok = bool(bound.max() < 2.0 ** 24 and np.array_equal(yu[:, cols].cpu().numpy(), ref.astype(np.float32)))
        del wu, yu
        return ok, engines

    def _performance(self, w, x, entry, M, N, K, wtype) -> dict:
        fn = lambda: ops.forward(w, x, M, N, K, entry=entry)  # noqa: E731
        for _ in range(self.warmup):
            fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(self.iterations):
            fn()
        e.record()
        e.synchronize()
        eager_ms = s.elapsed_time(e) / self.iterations
        # the same call from a HIP graph: the device time without host launch cost
        out = torch.empty((M, N), dtype=torch.float32, device=self.dev)
        wt, at = _lib.W_Q8_0, _lib.A_F32
        for k, v in ops.ENTRY_POINTS.items():
            if k == entry:
                wt, at = v
        reps = max(1, min(self.iterations, 20))
        gph = torch.cuda.CUDAGraph()
        ops.gemm(wt, at, w, x, M, N, K, out=out)
        torch.cuda.synchronize()
        with torch.cuda.graph(gph):
            for _ in range(reps):
                ops.gemm(wt, at, w, x, M, N, K, out=out)
        gph.replay()
        torch.cuda.synchronize()
        n_rep = max(1, self.iterations // reps)
        s.record()
        for _ in range(n_rep):
            gph.replay()
        e.record()
        e.synchronize()
        dev_ms = s.elapsed_time(e) / (n_rep * reps)
        del gph
        ops_count = 2.0 * M * N * K
        nbytes = N * (K // 32) * BLOCK_BYTES[wtype] + M * K * 4 + M * N * 4
        b = {"latency_ms": round(dev_ms, 6), "latency_ms_eager": round(eager_ms, 6),
             "tflops": round(ops_count / (dev_ms * 1e-3) / 1e12, 3),
             "gflops": round(ops_count / (dev_ms * 1e-3) / 1e9, 1),
             "gbps": round(nbytes / (dev_ms * 1e-3) / 1e9, 1)}
        base = ggml_baseline(wtype, N, M, K, self.hardware)
        if base:
            b["ggml"] = {"hardware": self.hardware, "tflops": base[0], "us_per_run": base[1]}
            b["vs_ggml_pct"] = round(100.0 * b["tflops"] / base[0], 1) if base[0] else None
        return b

    def _first_comparison(self, benches, wtype, cfgs, N, K):
        """The reference's baseline_comparison: the first configuration only (unified_test_runner.py:537-570)."""
        if not benches or "ggml" not in benches[0]:
            return None
        b = benches[0]
        ratio = b["vs_ggml_pct"]
        return {"current_hardware": torch.cuda.get_device_properties(0).name, "baseline_hardware": self.hardware,
                "current_tflops": b["tflops"], "baseline_tflops": b["ggml"]["tflops"],
                "performance_ratio": ratio, "better": bool(ratio is not None and ratio >= 100)}

    def _save(self, res: dict, attempt_dir: str | None) -> dict:
        if attempt_dir:
            os.makedirs(attempt_dir, exist_ok=True)
            with open(os.path.join(attempt_dir, "test_results.json"), "w") as f:
                json.dump(res, f, indent=2)
        return res


# ---------------------------------------------------------------- sweep over the definition table
def definitions_table() -> list[dict]:
    with open(os.path.join(DATA, "quant_gemm_definitions.json")) as f:
        return json.load(f)["definitions"]


def sweep(filter_text: str | None, runner: DefinitionRunner, out: str | None) -> dict:
    table = [d for d in definitions_table() if not filter_text or filter_text in d["name"]]
    summary, t0 = [], time.time()
    for i, d in enumerate(table):
        runner.log(f"[{i + 1}/{len(table)}] {d['name']} ({d['weight_dtype']}, N={d['N']}, K={d['K']})")
        r = runner.run(spec_from_table(d))
        for b in r["performance"].get("benchmarks", []):
            summary.append({"definition": d["name"], "weight": d["weight_dtype"].replace("block_", ""),
                            "N": d["N"], "K": d["K"], "config": b["config"],
                            "M": next(c["M"] for c in test_configs(spec_from_table(d), runner.all_configs)
                                      if c["name"] == b["config"]),
                            "us": round(b["latency_ms"] * 1e3, 2), "tflops": b["tflops"], "gbps": b["gbps"],
                            "ggml_tflops": (b.get("ggml") or {}).get("tflops"), "vs_ggml_pct": b.get("vs_ggml_pct")})
        if not r["correctness"].get("passed"):
            summary.append({"definition": d["name"], "failed": True,
                            "cases": r["correctness"].get("test_cases"), "errors": r["compilation"].get("errors")})
        torch.cuda.empty_cache()
    ok = [s for s in summary if not s.get("failed")]
    ratios = [s["vs_ggml_pct"] for s in ok if s.get("vs_ggml_pct")]
    result = {"definitions": len(table), "cases": len(ok), "failed": [s for s in summary if s.get("failed")],
              "baseline_hardware": runner.hardware,
              "geomean_vs_ggml_pct": round(float(np.exp(np.mean(np.log(ratios)))), 1) if ratios else None,
              "seconds": round(time.time() - t0, 1), "results": ok}
    if out:
        with open(out, "w") as f:
            json.dump(result, f, indent=1)
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--definition", help="definition JSON, operator spec.json or operator variant directory")
    ap.add_argument("--operators", help="operators directory (core/operators): run every discovered variant of "
                                        "its quant_gemm family, each in <attempt-path>/<variant>/")
    ap.add_argument("--attempt-path", help="directory for test_results.json")
    ap.add_argument("--sweep", action="store_true", help="run every definition of the built-in table")
    ap.add_argument("--filter", help="sweep only definitions whose name contains this text")
    ap.add_argument("--all-configs", action="store_true", help="the definition's test_configs, not M = 1, 8, 512")
    ap.add_argument("--baseline-hardware", default="RTX4090",
                    choices=["RTX4090", "A100", "A800", "H800", "RTX4070", "RTX5070"])
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--iterations", type=int, default=100)
    ap.add_argument("--out", help="sweep results JSON")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("ksq.runner needs a GPU (libksq has no CPU path)", file=sys.stderr)
        return 2
    runner = DefinitionRunner(args.warmup, args.iterations, args.baseline_hardware, args.all_configs,
                              log=lambda s: print(s, flush=True))
    if args.sweep:
        r = sweep(args.filter, runner, args.out)
        print(json.dumps({k: v for k, v in r.items() if k != "results"}), flush=True)
        return 0 if not r["failed"] else 1
    if args.operators:
        ok = True
        for v in discover(args.operators):
            out = os.path.join(args.attempt_path, v["_variant"]) if args.attempt_path else None
            r = runner.run(v, out)
            ok &= bool(r["correctness"].get("passed"))
            print(json.dumps({"variant": v["_variant"], "entry_point": r["compilation"].get("entry_point"),
                              "correctness": r["correctness"].get("passed"),
                              "benchmarks": r["performance"].get("benchmarks")}), flush=True)
        return 0 if ok else 1
    if not args.definition:
        ap.error("--definition, --operators or --sweep is required")
    r = runner.run(load_spec(args.definition), args.attempt_path)
    print(json.dumps({"compilation": r["compilation"].get("success"), "correctness": r["correctness"].get("passed"),
                      "benchmarks": r["performance"].get("benchmarks")}), flush=True)
    return 0 if r["correctness"].get("passed") else 1


if __name__ == "__main__":
    sys.exit(main())
