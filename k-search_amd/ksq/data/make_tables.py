"""Writes the two data tables the definition runner (ksq.runner) uses, from a KernelEvalPlus checkout.

    python k-search_amd/ksq/data/make_tables.py /root/reference/kernelevalplus-main

quant_gemm_definitions.json
    one entry per quant_gemm definition file (kernelevalplus-main/definitions/quant_gemm/**/*.json):
    its name, weight / activation dtypes, the constant N and K axes, the M values of its
    test_configs, its accuracy threshold (null when the definition leaves it to the runner's
    default) and its model architectures.  The runner needs the shapes and names only, so
    the descriptions, tags and formula text are not carried.
ggml_baseline_quant_gemm.json
    the GGML (llama.cpp test-backend-ops MUL_MAT) timings the reference compares against
    (kernelevalplus-main/data/baseline/baseline_data_compact.json, read through
    core/tools/baseline_api.py), restricted to the (type, N, M, K) cases of those
    definitions.  Keys keep the reference's case ids ("w4a32c8_q4_0_f32_m{N}_n{M}_k{K}":
    GGML's m is the output features, n the batch), values {hardware: [tflops, us_per_run]}.

Run in a container that has the reference; the tables are committed, so nothing reads
the reference at run time.
"""
from __future__ import annotations

import glob
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HARDWARE = ("RTX4090", "A100", "A800", "H800", "RTX4070", "RTX5070")


def main(kep_root: str) -> None:
    files = sorted(glob.glob(os.path.join(kep_root, "definitions", "quant_gemm", "**", "*.json"), recursive=True))
    defs = []
    for f in files:
        with open(f) as fh:
            d = json.load(fh)
        if d.get("op_type") != "quant_gemm":
            continue
        acc = d.get("accuracy") or {}
        defs.append({
            "name": d["name"][:-5] if d["name"].endswith(".json") else d["name"],
            "path": os.path.relpath(f, kep_root),
            "weight_dtype": d["inputs"]["weight"]["dtype"],
            "activation_dtype": d["inputs"]["activation"]["dtype"],
            "N": d["axes"]["N"]["value"],
            "K": d["axes"]["K"]["value"],
            "M": [c["M"] for c in d.get("test_configs", [])],
            "threshold": acc.get("threshold"),
            "models": d.get("model_architectures", []),
        })
    with open(os.path.join(HERE, "quant_gemm_definitions.json"), "w") as fh:
        json.dump({"source": "kernelevalplus-main/definitions/quant_gemm", "definitions": defs}, fh, indent=1)

    with open(os.path.join(kep_root, "data", "baseline", "baseline_data_compact.json")) as fh:
        base = json.load(fh)
    table = {}
    for d in defs:
        t = d["weight_dtype"].replace("block_", "")
        bits = "4" if t.startswith("q4") else "8"
        for M in d["M"]:
            key = f"w{bits}a32c8_{t}_f32_m{d['N']}_n{M}_k{d['K']}"
            entry = base.get(key)
            if not isinstance(entry, dict) or "hardware" not in entry:
                continue
            hw = {}
            for h in HARDWARE:
                v = entry["hardware"].get(h)
                if v and v.get("tflops") is not None:
                    us = v.get("us_per_run")
                    if us is None and v.get("latency_ms") is not None:
                        us = v["latency_ms"] * 1000.0
                    hw[h] = [v["tflops"], us]
            table[key] = hw
    with open(os.path.join(HERE, "ggml_baseline_quant_gemm.json"), "w") as fh:
        fh.write('{"source": "kernelevalplus-main/data/baseline/baseline_data_compact.json",\n')
        fh.write(' "value": "[tflops, us_per_run]",\n "cases": {\n')
        fh.write(",\n".join(f"  {json.dumps(k)}: {json.dumps(table[k], sort_keys=True)}" for k in sorted(table)))
        fh.write("\n }\n}\n")
    print(f"{len(defs)} definitions, {len(table)} baseline cases written to {HERE}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/kernelevalplus-main")
