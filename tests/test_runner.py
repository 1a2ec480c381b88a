"""The definition runner (ksq.runner) and its checker (ksq.refcheck).  CPU parts here;
the end-to-end run of definitions is in test_gpu_parity.py.

refcheck is the runner's own restatement of the exact checks; it is pinned here against
the C oracle (bit-exact where the oracle is bit-exact, 1e-12 for the fp64 formulas)."""
import json
import os

import numpy as np
import pytest
import torch

import npref

LEGACY = (0, 1, 4, 5, 6)


def test_refcheck_quantize_q8_1_matches_oracle(oracle):
    from ksq import refcheck
    g = np.random.default_rng(3000)
    x = g.standard_normal((12, 512), dtype=np.float32)
    x[2, :32] = 0.0
    x[4, :8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5, 3.49999976]
    x[4, 8:32] = 0.0
    assert np.array_equal(refcheck.quantize_q8_1(x), oracle.quantize_q8_1(x))
    assert np.array_equal(refcheck.quantize_q8s(x), oracle.quantize_q8s(x))


@pytest.mark.parametrize("wtype", LEGACY)
def test_refcheck_block_formulas_match_oracle(oracle, wtype):
    from ksq import refcheck, synth
    g = np.random.default_rng(3010 + wtype)
    M, N, K = 3, 9, 512
    w = synth.weights(wtype, g, N, K)
    a = oracle.quantize_q8_1(synth.activations(g, M, K))
    assert np.array_equal(refcheck.block_sumi(wtype, a, w), oracle.block_sumi(wtype, a, w, M, N, K))
    ref = oracle.gemm_f64(wtype, a, w, M, N, K)
    assert np.allclose(refcheck.gemm_f64(wtype, a, w), ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())
    deq = oracle.dequantize(wtype, w.reshape(N, -1), N, K)
    assert np.array_equal(refcheck.dequantize(wtype, w).astype(np.float32), deq)
    if wtype == 1:
        a8 = oracle.quantize_q8s(synth.activations(g, M, K))
        r8 = oracle.gemm_q8s_f64(a8, w, M, N, K)
        assert np.allclose(refcheck.gemm_q8s_f64(a8, w), r8, rtol=1e-12, atol=1e-12 * np.abs(r8).max())


def test_refcheck_max_rel_err_floor():
    from ksq import refcheck
    ref = np.array([[1.0, 1e-9, -2.0]])
    assert refcheck.max_rel_err(ref, ref) == 0.0
    assert abs(refcheck.max_rel_err(ref + [[0, 1e-6, 0]], ref) - 1e-6 / 2e-3) < 1e-12


@pytest.mark.parametrize("wtype", LEGACY)
def test_runner_weight_quantisers(oracle, wtype):
    """The runner's device-side input quantisers (torch, here on the CPU): Q4_1 byte-equal to the
    harness quantize_to_q4_1 restatement, Q5_x byte-equal to the oracle's GGML encoders, every type
    within half a step after dequantisation (torch dequantiser == oracle dequantiser)."""
    from ksq import runner
    g = np.random.default_rng(3100 + wtype)
    N, K = 6, 256
    wf = g.standard_normal((N, K), dtype=np.float32)
    wf[1, :32] = 0.0
    w = runner.quantize_weights(torch.from_numpy(wf), wtype).numpy()
    assert w.shape == (N, K // 32, {0: 18, 1: 34, 4: 20, 5: 22, 6: 24}[wtype])
    if wtype == 4:
        assert np.array_equal(w, npref.quantize_q4_1(wf))
    if wtype == 5:
        assert np.array_equal(w, oracle.quantize_q5_0(wf))
    if wtype == 6:
        assert np.array_equal(w, oracle.quantize_q5_1(wf))
    deq = runner.dequantize_weights(torch.from_numpy(w), wtype).numpy()
    assert np.array_equal(deq, oracle.dequantize(wtype, w.reshape(N, -1), N, K))
    xb, yb = wf.reshape(-1, 32), deq.reshape(-1, 32)
    span = np.abs(xb).max(1) if wtype in (0, 1, 5) else xb.max(1) - xb.min(1)
    steps = {0: 7, 1: 127, 4: 15, 5: 16, 6: 31}[wtype]
    slack = 1.0 if wtype in (0, 5) else 0.5      # symmetric 4/5-bit ranges lose a step at one end
    assert np.all(np.abs(xb - yb).max(1) <= span / steps * slack + 3e-3 * np.abs(xb).max(1) + 1e-7)


def test_runner_spec_handling(tmp_path):
    from ksq import _lib, runner
    table = runner.definitions_table()
    assert len(table) == 87
    assert {d["weight_dtype"].replace("block_", "") for d in table} == {"q4_0", "q4_1", "q8_0"}
    d = next(t for t in table if t["name"] == "w4a32c8_q4_1_fp32_int8_qwen3_4b_att_out_n2560_k2560")
    spec = runner.spec_from_table(d)
    assert runner.resolve(spec) == (_lib.W_Q4_1, _lib.A_F32, "gemm_w4a32c8_q4_1_fp32_int8")
    assert [c["M"] for c in runner.test_configs(spec, False)] == [1, 8, 512]
    assert [c["M"] for c in runner.test_configs(spec, True)] == [1, 2, 3, 4, 5, 8, 512]
    assert all(c["N"] == 2560 and c["K"] == 2560 for c in runner.test_configs(spec, True))
    # a definition file in the reference's own form (axes, inputs, test_configs)
    p = tmp_path / "def.json"
    p.write_text(json.dumps({"name": "w8a32c8_q8_0_fp32_int8_x_n4096_k4096", "op_type": "quant_gemm",
                             "axes": {"M": {"type": "var"}, "N": {"type": "const", "value": 4096},
                                      "K": {"type": "const", "value": 4096}},
                             "inputs": {"weight": {"dtype": "block_q8_0"}, "activation": {"dtype": "float32"}},
                             "test_configs": [{"name": "batch_1", "M": 1, "N": 4096, "K": 4096}]}))
    s = runner.load_spec(str(p))
    assert s["params"]["N"] == {"value": 4096} and s["params"]["M"] == {"default": 1}
    assert runner.resolve(s)[2] == "gemm_w8a32c8_q8_0_fp32_int8"
    native = {"name": "w8a8c8_q8_0_q8_1", "kernel": {"entry_point": "gemm_w8a8c8_q8_0_q8_1"},
              "inputs": {"weight": {"dtype": "block_q8_0"}, "activation": {"dtype": "float32"}},
              "params": {"N": {"default": 7168}, "K": {"default": 7168}}}
    assert runner.resolve(native) == (_lib.W_Q8_0, _lib.A_F32_Q8S, "gemm_w8a8c8_q8_0_q8_1")
    assert [(c["M"], c["N"], c["K"]) for c in runner.test_configs(native, False)] == [
        (1, 7168, 7168), (8, 7168, 7168), (512, 7168, 7168)]
    with pytest.raises(ValueError):
        runner.resolve({"inputs": {"weight": {"dtype": "q4_0"}, "activation": {"dtype": "block_q8_1"}}})


# the deepseek_v2 operator's identifying fields (core/operators/quant_gemm/variants/deepseek_v2/
# w4a32c8_q4_0_fp32_int8/spec.json): the generic operator's name, entry "forward", one architecture
DSV2_SPEC = {"name": "w4a32c8_q4_0_fp32_int8", "variant": "W4A32C8", "family": "quant_gemm",
             "model_architectures": ["deepseek-v2"], "kernel": {"file": "kernel.cu", "entry_point": "forward"},
             "inputs": {"weight": {"dtype": "block_q4_0"}, "activation": {"dtype": "float32"}},
             "params": {"M": {"type": "int"}, "N": {"type": "int", "default": 5120},
                        "K": {"type": "int", "default": 5120}},
             "test_configs": [{"name": f"batch_{m}", "M": m} for m in (1, 2, 3, 4, 5, 8, 512)],
             "accuracy": {"metric": "nmse", "threshold": 0.1}}


def test_runner_resolves_variant_identity():
    """The entry a spec resolves to follows its identity, not its weight dtype alone: the
    deepseek_v2 W4A32C8 spec (entry "forward") runs the block_q8f entry with fp32 d_a and s_a; the
    same name without the architecture runs the generic gemm_{name}; the reference's order
    (entry_point, gemm_{name}, name) picks the native W8A8C8 entry either way."""
    from ksq import _lib, runner
    assert runner.entry_candidates(DSV2_SPEC)[:2] == ["gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2", "forward_deepseek_v2"]
    assert runner.resolve(DSV2_SPEC) == (_lib.W_Q4_0, _lib.A_F32_Q8F_RNE, "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2")
    generic = {k: v for k, v in DSV2_SPEC.items() if k != "model_architectures"}
    assert runner.resolve(generic) == (_lib.W_Q4_0, _lib.A_F32, "gemm_w4a32c8_q4_0_fp32_int8")
    # the architecture can also come from the variant directory the spec was found under
    by_dir = dict(generic, _variant_dir="/x/quant_gemm/variants/deepseek_v2/w4a32c8_q4_0_fp32_int8")
    assert runner.resolve(by_dir)[2] == "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2"
    native = {"name": "w8a8c8_q8_0_q8_1", "model_architectures": ["deepseek-v3"],
              "kernel": {"entry_point": "forward"},
              "inputs": {"weight": {"dtype": "block_q8_0"}, "activation": {"dtype": "float32"}}}
    assert runner.resolve(native) == (_lib.W_Q8_0, _lib.A_F32_Q8S, "gemm_w8a8c8_q8_0_q8_1")
    # an entry whose weight type contradicts the spec's weight dtype is refused
    with pytest.raises(ValueError):
        runner.resolve(dict(native, inputs={"weight": {"dtype": "block_q4_0"}, "activation": {"dtype": "float32"}}))


def _write_family(root, variants):
    fam = root / "quant_gemm"
    (fam / "variants").mkdir(parents=True)
    (fam / "manifest.json").write_text(json.dumps({"name": "quant_gemm", "op_type": "gemm"}))
    for rel, spec, impl in variants:
        d = fam / "variants" / rel
        d.mkdir(parents=True)
        (d / "spec.json").write_text(json.dumps(spec))
        if impl is not None:
            (d / "impl.json").write_text(json.dumps(impl))
    return fam


def test_runner_discovers_variant_directories(tmp_path):
    """discover() walks <family>/manifest.json and variants/**/spec.json as the reference's
    OperatorRegistry does (plus the nested variants/<model>/<variant>/ layout), merges impl.json's
    kernel entry, and each discovered variant resolves to its own libksq entry."""
    from ksq import _lib, runner
    dsv2 = {k: v for k, v in DSV2_SPEC.items() if k != "model_architectures"}   # identity from the path only
    dsv3 = {"name": "w8a8c8_q8_0_q8_1", "inputs": {"weight": {"dtype": "block_q8_0"},
                                                    "activation": {"dtype": "float32"}}}
    plain = {"name": "w8a32c8_q8_0_fp32_int8", "inputs": {"weight": {"dtype": "block_q8_0"},
                                                          "activation": {"dtype": "float32"}}}
    _write_family(tmp_path, [
        ("deepseek_v2/w4a32c8_q4_0_fp32_int8", dsv2, {"name": "w4a32c8_q4_0_fp32_int8"}),
        ("deepseek_v3/w8a8c8_q8_0_q8_1", dsv3, {"kernel": {"file": "kernel.cu", "entry_point": "gemm_w8a8c8_q8_0_q8_1"}}),
        ("w8a32c8_q8_0_fp32_int8", plain, None)])
    found = runner.discover(str(tmp_path))
    got = {v["_variant"]: runner.resolve(v) for v in found}
    assert got == {
        "deepseek_v2/w4a32c8_q4_0_fp32_int8": (_lib.W_Q4_0, _lib.A_F32_Q8F_RNE, "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2"),
        "deepseek_v3/w8a8c8_q8_0_q8_1": (_lib.W_Q8_0, _lib.A_F32_Q8S, "gemm_w8a8c8_q8_0_q8_1"),
        "w8a32c8_q8_0_fp32_int8": (_lib.W_Q8_0, _lib.A_F32, "gemm_w8a32c8_q8_0_fp32_int8")}
    v3 = next(v for v in found if v["_variant"].startswith("deepseek_v3"))
    assert v3["kernel"]["entry_point"] == "gemm_w8a8c8_q8_0_q8_1" and "_impl" in v3
    # a variant directory given directly loads the same spec
    d = runner.load_spec(str(tmp_path / "quant_gemm" / "variants" / "deepseek_v2" / "w4a32c8_q4_0_fp32_int8"))
    assert runner.resolve(d)[2] == "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2"
    with pytest.raises(FileNotFoundError):
        runner.discover(str(tmp_path / "quant_gemm"))


REF_OPERATORS = "/root/reference/kernelevalplus-main/core/operators"


@pytest.mark.skipif(not os.path.isdir(REF_OPERATORS), reason="the reference tree is not on this machine")
def test_runner_resolves_reference_operator_specs():
    """The reference's own quant_gemm operator variants (read as JSON data) resolve to the libksq
    entries with their arithmetic: deepseek_v2 to the block_q8f entry, deepseek_v3 to the native
    W8A8C8 symbol."""
    from ksq import _lib, runner
    got = {v["_variant"]: runner.resolve(v) for v in runner.discover(REF_OPERATORS)}
    assert got["deepseek_v2/w4a32c8_q4_0_fp32_int8"] == (_lib.W_Q4_0, _lib.A_F32_Q8F_RNE,
                                                         "gemm_w4a32c8_q4_0_fp32_int8_deepseek_v2")
    assert got["deepseek_v3/w8a8c8_q8_0_q8_1"] == (_lib.W_Q8_0, _lib.A_F32_Q8S, "gemm_w8a8c8_q8_0_q8_1")


@pytest.mark.parametrize("rule", [0, 1])
def test_refcheck_quantize_q8f_matches_oracle(oracle, rule):
    """The runner's numpy block_q8f quantiser equals the oracle's C restatement bit for bit, on
    random rows, exact ties of x / d (x = k + 0.5 with amax 127: d = 1), a zero block and tiny
    blocks."""
    from ksq import refcheck
    g = np.random.default_rng(31 + rule)
    x = g.standard_normal((6, 256), dtype=np.float32) * np.float32(3.0)
    x[1, :32] = np.arange(-16, 16, dtype=np.float32) + np.float32(0.5)
    x[1, 31] = np.float32(127.0)
    x[2, 32:64] = 0.0
    x[3, 64:96] *= np.float32(1e-12)
    assert np.array_equal(refcheck.quantize_q8f(x, rule), oracle.quantize_q8f(x, rule))


def test_runner_ggml_table():
    from ksq import _lib, runner
    # the GGML rows quoted for config 0 and config 1 (RTX 4090 / H800)
    assert runner.ggml_baseline(_lib.W_Q4_0, 4096, 1, 4096, "RTX4090") == [4.95, 6.77]
    assert runner.ggml_baseline(_lib.W_Q4_0, 4096, 1, 4096, "H800") == [3.8, 8.83]
    assert runner.ggml_baseline(_lib.W_Q8_0, 4096, 8, 4096, "RTX4090")[0] == 14.23
    assert runner.ggml_baseline(_lib.W_Q4_0, 4096, 2048, 4096, "RTX4090") is None
    # every definition configuration has a GGML row
    for d in runner.definitions_table():
        wt = runner.resolve(runner.spec_from_table(d))[0]
        for M in d["M"]:
            assert runner.ggml_baseline(wt, d["N"], M, d["K"], "RTX4090") is not None, (d["name"], M)


def test_runner_without_gpu_exits_cleanly(monkeypatch, capsys):
    from ksq import runner
    monkeypatch.setattr(torch.cuda, "is_available", lambda: False)
    assert runner.main(["--sweep"]) == 2
    assert "needs a GPU" in capsys.readouterr().err
