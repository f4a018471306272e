"""Write tests/golden/ref_logits.json and ref_gemma4.json from the
reference's llama.cpp golden rows.

Run once in the build container (it reads /root/reference as text; nothing
at test time does). Sources: test/test_qwen_moe.lua:202-305 (REF.<arch>,
IDX, batches, N_DECODE, TOL) and test/test_gemma4.lua:174-224,298-300
(REF.dense, IDX, batches, N_DECODE, the CPU TOL). Each row: input id,
argmax ("best"), logits at the 1-based IDX.
"""
import json
import os
import re
import sys

REF = "/root/reference/test"


def parse_rows(text, name):
    m = re.search(r"^REF\.%s = \{\n(.*?)^\}" % re.escape(name), text, re.S | re.M)
    if not m:
        return None
    rows = []
    for line in m.group(1).splitlines():
        r = re.search(r"id = (\d+), best = (\d+), v = \{ ([^}]*) \}", line)
        if r:
            rows.append({"id": int(r.group(1)), "best": int(r.group(2)),
                         "v": [float(x) for x in r.group(3).split(",")]})
    return rows


def main(out):
    text = open(os.path.join(REF, "test_qwen_moe.lua")).read()
    idx = [int(x) for x in re.search(r"local IDX = \{ ([^}]*) \}", text).group(1).split(",")]
    batches = [[int(x) for x in b.split(",")] for b in
               re.findall(r"\{ ([\d, ]+) \}", re.search(r"local batches = (\{.*?\}\s*\})\n", text).group(1))]
    ndec = int(re.search(r"local N_DECODE = (\d+)", text).group(1))
    tol = float(re.search(r"local TOL = ([0-9.e-]+)", text).group(1))
    data = {"source": "test/test_qwen_moe.lua:202-305", "idx_1based": idx, "batches": batches,
            "n_decode": ndec, "tol": tol, "rows": {}}
    for arch in ("llama", "qwen3", "qwen3moe"):
        data["rows"][arch] = parse_rows(text, arch)
    with open(out, "w") as f:
        json.dump(data, f, indent=1)


def main_gemma4(out):
    text = open(os.path.join(REF, "test_gemma4.lua")).read()
    idx = [int(x) for x in re.search(r"local IDX = \{ ([^}]*) \}", text).group(1).split(",")]
    batches = [[int(x) for x in b.split(",")] for b in
               re.findall(r"\{ ([\d, ]+) \}", re.search(r"local batches = (\{.*?\n\})\n", text, re.S).group(1))]
    ndec = int(re.search(r"local N_DECODE = (\d+)", text).group(1))
    # "local TOL, LOOSE = GPU and 2e-2 or 2e-3, ...": the CPU tolerance
    tol = float(re.search(r"local TOL, LOOSE = GPU and [0-9.e-]+ or ([0-9.e-]+)", text).group(1))
    data = {"source": "test/test_gemma4.lua:174-224,298-300", "idx_1based": idx,
            "batches": batches, "n_decode": ndec, "tol": tol,
            "rows": {"dense": parse_rows(text, "dense")}}
    with open(out, "w") as f:
        json.dump(data, f, indent=1)


if __name__ == "__main__":
    here = os.path.dirname(__file__)
    main(sys.argv[1] if len(sys.argv) > 1 else os.path.join(here, "ref_logits.json"))
    main_gemma4(sys.argv[2] if len(sys.argv) > 2 else os.path.join(here, "ref_gemma4.json"))
