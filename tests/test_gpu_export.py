"""GGUF export / load and training checkpoints on the GPU (tests/js/export.mjs):
loadGGUF(exportGGUF(w)) decodes bit-identically to loading w directly, and
training resumed from saveCheckpoint / loadCheckpoint is bit-identical to
training that never stopped (losses, gradient norms, parameters, Adam m/v)."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.gpu
def test_export_and_checkpoint_js(fh):
    r = subprocess.run(["node", os.path.join(ROOT, "tests", "js", "export.mjs")], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=600)
    res = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    for x in res:
        print(x["test"], "ok" if x["ok"] else "FAIL", x.get("detail") or x.get("error", ""))
    assert r.returncode == 0 and len(res) == 5 and all(x["ok"] for x in res), r.stdout[-4000:]
