"""The step's TunableOp results for its plain GEMMs (step.use_tuned_gemms): the
file's validators match the runtime on MI355X, the tuned solutions give the
library default's products (bf16 GEMMs with fp32 accumulation: within 1e-2
relative L2 of fp32, and within 5e-3 of the default's own result), and a
process that reads the file writes no TunableOp results of its own."""

import subprocess
import sys
from pathlib import Path

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

SHAPES = [(1024, 1536), (1024, 1024), (1024, 6144), (3072, 1024), (1024, 151936)]  # (in, out) at 8192 tokens


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm())


def test_tuned_gemms_match_the_default():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    from voodoo_quant.training import step as st

    g = torch.Generator(device="cuda").manual_seed(3)
    cases = []
    for din, dout in SHAPES:
        x = torch.randn(8192, din, device="cuda", generator=g).to(torch.bfloat16)
        w = (torch.randn(dout, din, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        cases.append((x, w, F.linear(x, w)))
    torch.cuda.synchronize()
    try:
        assert st.use_tuned_gemms(), "validators of the tuning file differ from this runtime"
        for (x, w, y0), (din, dout) in zip(cases, SHAPES):
            y1 = F.linear(x, w)
            ref = x.float() @ w.float().t() if dout < 100000 else None
            err_default = _rel(y1, y0)
            print(f"[tuned] {din}->{dout}: tuned vs default {err_default:.2e}", flush=True)
            assert err_default < 5e-3
            if ref is not None:
                assert _rel(y1, ref) < 1e-2
    finally:
        torch.cuda.tunable.enable(False)


def test_reading_the_tuning_file_writes_no_results(tmp_path):
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    pkg = Path(__file__).resolve().parent.parent / "voodoo-dyn-quant_amd"
    code = ("import sys, torch, torch.nn.functional as F; sys.path.insert(0, %r); "
            "from voodoo_quant.training import step as st; assert st.use_tuned_gemms(); "
            "x = torch.randn(8192, 1024, device='cuda').to(torch.bfloat16); "
            "w = torch.randn(1536, 1024, device='cuda').to(torch.bfloat16); "
            "F.linear(x, w); torch.cuda.synchronize(); print('ok')" % str(pkg))
    res = subprocess.run([sys.executable, "-c", code], cwd=tmp_path, capture_output=True, text=True, timeout=110)
    assert res.returncode == 0 and "ok" in res.stdout, res.stderr[-2000:]
    assert not list(tmp_path.glob("tunableop*")), list(tmp_path.iterdir())
