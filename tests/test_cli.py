"""JSON-in / JSON-out CLI of the lowering (role of intentir_cuda_codegen --intent --bindings)."""

from __future__ import annotations

import json
import subprocess
import sys

import numpy as np
import pytest

from intent_ir_amd.cli import lower_from_json_str, main
from intent_ir_amd.configs import WORKLOADS
from tests.ew_cases import CASES


def _write(tmp_path, name, obj):
    p = tmp_path / name
    p.write_text(json.dumps(obj))
    return str(p)


@pytest.mark.parametrize("key", sorted(WORKLOADS))
def test_cli_lowers_every_workload(tmp_path, capsys, key):
    w = WORKLOADS[key]
    rc = main(["--intent", _write(tmp_path, "i.json", w.ir()), "--bindings", _write(tmp_path, "b.json", w.bindings)])
    assert rc == 0
    out = json.loads(capsys.readouterr().out)
    assert out["kernel_id"].startswith("ihip_")
    assert set(out) >= {"kernel_name", "io_spec", "launch", "output_names", "bindings", "call_args"}
    assert out == json.loads(lower_from_json_str(json.dumps(w.ir()), json.dumps(w.bindings)))


def test_cli_spells_out_elementwise_programs(tmp_path, capsys):
    name, ir, b, _ = next(c for c in CASES if c[0] == "two_outputs_shared")
    assert main(["--intent", _write(tmp_path, "i.json", ir), "--bindings", _write(tmp_path, "b.json", b)]) == 0
    out = json.loads(capsys.readouterr().out)
    prog = out["call_args"][0]
    assert out["kernel_id"] == "ihip_elementwise_program" and prog["kind"] == "ew_program"
    assert prog["outputs"] == ["y1", "y2"] and prog["shape"] == [9, 40]
    assert all(len(c) == 6 for c in prog["code"]) and prog["listing"][-1].startswith("y2 = ")


def test_cli_exit_codes(tmp_path, capsys):
    assert main([]) == 2
    assert main(["--intent", "x.json"]) == 2
    bad = {"name": "g", "tensors": {"x": {"dtype": "f32", "shape": ["N"]}, "i": {"dtype": "i32", "shape": ["N"]},
                                    "y": {"dtype": "f32", "shape": ["N"]}},
           "ops": [{"op": "gather", "inputs": ["x", "i"], "output": "y"}], "outputs": ["y"]}
    rc = main(["--intent", _write(tmp_path, "i.json", bad), "--bindings", _write(tmp_path, "b.json", {"N": 4})])
    assert rc == 3 and "unsupported" in capsys.readouterr().err
    rc = main(["--intent", str(tmp_path / "missing.json"), "--bindings", _write(tmp_path, "b.json", {})])
    assert rc == 3
    invalid = {"name": "v", "tensors": {"x": {"dtype": "f32", "shape": ["N"]}},
               "ops": [{"op": "exp", "inputs": ["nope"], "output": "x"}], "outputs": ["x"]}
    rc = main(["--intent", _write(tmp_path, "v.json", invalid), "--bindings", _write(tmp_path, "b.json", {"N": 4})])
    assert rc == 3 and "undefined tensor" in capsys.readouterr().err


def test_cli_as_a_process(tmp_path):
    w = WORKLOADS["softmax"]
    res = subprocess.run([sys.executable, "-m", "intent_ir_amd.cli", "--intent", _write(tmp_path, "i.json", w.ir()),
                          "--bindings", _write(tmp_path, "b.json", {"M": 4, "N": 64})], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    assert json.loads(res.stdout)["kernel_id"] == "ihip_softmax_rows_f32"


@pytest.mark.gpu
def test_cli_run_on_gpu(hip, tmp_path):
    from oracle.interpreter import execute_intent

    w = WORKLOADS["softmax"]
    b = {"M": 8, "N": 1024}
    inp = w.gen(b)
    np.savez(tmp_path / "in.npz", **inp)
    rc = main(["--intent", _write(tmp_path, "i.json", w.ir()), "--bindings", _write(tmp_path, "b.json", b),
               "--run", str(tmp_path / "in.npz"), "--out", str(tmp_path / "out.npz")])
    assert rc == 0
    with np.load(tmp_path / "out.npz") as z:
        got = z["output_ptr"]
    ref = execute_intent(w.ir(), inp, b)["output_ptr"]
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-7)
