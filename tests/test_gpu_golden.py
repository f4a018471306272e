"""The reference's own golden rows through the HIP path (lgmlh_forward).

REF.llama / REF.qwen3 / REF.qwen3moe (test/test_qwen_moe.lua:202-273, fixture
tests/golden/ref_logits.json): the tiny models of test_qwen_moe.lua:41-66
(E 64, 4 query / 2 KV heads of 16, f32 weights, vocab 259) regenerated with
the reference's LCG and draw order, run on the GPU over the golden passes
(two prompt batches, then 6 greedy decode ids), every token's logits at the
8 golden vocab indices within TOL 2e-3 (absolute, the reference's own
tolerance, test_qwen_moe.lua:378-400) and the argmax of every row equal to
the reference's `best`. These rows come from llama.cpp, so parity here does
not pass through this build's oracle; the oracle's rows are compared too.
The same models written as gguf files in the reference's layout and read
back by runtime.load_gguf meet the same rows on the device.
"""
import json
import os

import numpy as np
import pytest

from oracle import core, models
from tests.gpu_util import rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ref_logits.json")


def gpu_rows(arch, gm=None):
    from lgml_amd import runtime
    if gm is None:
        hp, w = models.ref_tiny(arch)
        gm = runtime.DeviceModel(hp, w, 128)
    d = json.load(open(GOLDEN))
    ref = d["rows"][arch]
    nb = sum(len(b) for b in d["batches"])
    passes = d["batches"] + [[r["id"]] for r in ref[nb:]]
    rows, npast = [], 0
    for ids in passes:
        ids = np.array(ids, np.int32)
        plan = gm.plan([len(ids)], [npast], np.array([[0, 1]], np.int32), ids)
        lg = gm.forward(plan, out_rows=np.arange(len(ids))).cpu().numpy()
        rows.extend(lg)
        npast += len(ids)
    return d, ref, rows


def check_rows(arch, d, ref, rows):
    idx = [i - 1 for i in d["idx_1based"]]
    assert len(rows) == len(ref) == 14
    err = 0.0
    for r, got in zip(ref, rows):
        err = max(err, max(abs(float(got[i]) - v) for i, v in zip(idx, r["v"])))
        assert int(np.argmax(got)) == r["best"], "argmax differs from llama.cpp"
    print("%s: max |logit - llama.cpp| %.3g (tol %g)" % (arch, err, d["tol"]), flush=True)
    assert err < d["tol"], "max logit error %.3g" % err


@pytest.mark.parametrize("arch", ["llama", "qwen3", "qwen3moe"])
def test_hip_path_matches_llama_cpp_rows(arch):
    from tests.test_oracle_golden import run_rows
    d, ref, rows = gpu_rows(arch)
    check_rows(arch, d, ref, rows)
    _, _, orows = run_rows(arch)
    assert rel_err(np.array(rows), np.array(orows)) < 1e-4


@pytest.mark.parametrize("arch", ["llama", "qwen3", "qwen3moe"])
def test_gguf_loaded_models_match_llama_cpp_rows(tmp_path, arch):
    """§8(f) row 3 end to end on the device: the tiny models written as gguf
    files with the reference's key-values and tensor names
    (test/test_qwen_moe.lua:65-200), read by runtime.load_gguf into a
    DeviceModel, meet the same llama.cpp rows."""
    from lgml_amd import runtime
    from tests import gguf_util as gw
    from tests.test_gguf_loader import kv_qwen, tensors_of
    hp, w = models.ref_tiny(arch)
    path = str(tmp_path / ("%s.gguf" % arch))
    gw.write(path, kv_qwen(arch, hp), tensors_of(arch, hp, w))
    d, ref, rows = gpu_rows(arch, runtime.load_gguf(path, 128))
    check_rows(arch, d, ref, rows)


GOLDEN_G4 = os.path.join(os.path.dirname(__file__), "golden", "ref_gemma4.json")


def test_hip_path_matches_gemma4_rows():
    """REF.dense of test/test_gemma4.lua:192-224 on the GPU: the tiny gemma4
    model (test_gemma4.lua:38-174) with a sliding layer (window 6, heads of
    16, 2 KV heads, through a ring) and a global one (heads of 32, 1 KV
    head, V = the raw K, proportional rope), post norms, GeGLU, output
    scales, tied output and a logit softcap; every token's logits at the
    golden indices within 2e-3 of llama.cpp and the argmax of every row."""
    from lgml_amd import runtime
    from tests.test_oracle_golden import run_gemma4_rows
    hp, w = models.ref_tiny_gemma4()
    rows = gemma4_rows(runtime.DeviceModel(hp, w, 128, ring_cells=64))
    _, _, orows = run_gemma4_rows()
    assert rel_err(np.array(rows), np.array(orows)) < 1e-4


def test_gguf_loaded_gemma4_matches_llama_cpp_rows(tmp_path):
    """The tiny gemma4 model as a gguf file (test/test_gemma4.lua:84-174:
    per-layer KV head counts, head sizes of 16 and 32, no attn_v on the
    global layer, tied output), read by runtime.load_gguf, meets REF.dense
    on the device."""
    from lgml_amd import runtime
    from tests import gguf_util as gw
    from tests.test_gguf_loader import kv_gemma4, tensors_of
    hp, w = models.ref_tiny_gemma4()
    path = str(tmp_path / "gemma4.gguf")
    gw.write(path, kv_gemma4(hp, w), tensors_of("gemma4", hp, w, gemma=True))
    gemma4_rows(runtime.load_gguf(path, 128, ring_cells=64))


def gemma4_rows(gm):
    d = json.load(open(GOLDEN_G4))
    ref = d["rows"]["dense"]
    nb = sum(len(b) for b in d["batches"])
    passes = d["batches"] + [[r["id"]] for r in ref[nb:]]
    rows, npast = [], 0
    for ids in passes:
        ids = np.array(ids, np.int32)
        plan = gm.plan([len(ids)], [npast], np.array([[0, 1]], np.int32), ids,
                       ring_tab=np.array([[0]], np.int32))
        rows.extend(gm.forward(plan, out_rows=np.arange(len(ids))).cpu().numpy())
        npast += len(ids)
    idx = [i - 1 for i in d["idx_1based"]]
    assert len(rows) == len(ref) == 31
    err = 0.0
    for r, got in zip(ref, rows):
        err = max(err, max(abs(float(got[i]) - v) for i, v in zip(idx, r["v"])))
        assert int(np.argmax(got)) == r["best"], "argmax differs from llama.cpp"
    print("gemma4 dense: max |logit - llama.cpp| %.3g (tol %g)" % (err, d["tol"]), flush=True)
    assert err < d["tol"], "max logit error %.3g" % err
    return rows
