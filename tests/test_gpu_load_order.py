"""Library loaded before torch.

PyTorch-ROCm wheels bundle their own HIP runtime. The package's loader
imports torch before it loads libfav4_bshd.so, so the library binds to
torch's runtime. This test runs a fresh process that loads the library
first and only then uses torch. The process must hold one libamdhip64, and
the forward must run. Without the loader's import the process held two
runtimes, and the first launch returned hipErrorNoDevice (100).
"""
import subprocess
import sys

import pytest

from tests.conftest import ROOT

pytestmark = pytest.mark.gpu

CODE = r"""
import sys
sys.path.insert(0, {root!r})
import __graft_entry__ as g
runner = g.import_package().Runner()
import torch
maps = sorted({{ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln}})
q = torch.randn(1, 64, 2, 128, device="cuda").to(torch.bfloat16)
o = torch.full_like(q, float("nan"))
runner.call(q, q, q, o, None, False, 0)
torch.cuda.synchronize()
print("runtimes", len(maps), "finite", bool(torch.isfinite(o.float()).all()))
"""


def test_library_loaded_before_torch_shares_its_runtime():
    print("  fresh process: package first, then torch", flush=True)
    out = subprocess.run([sys.executable, "-c", CODE.format(root=str(ROOT))], capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    assert out.stdout.split()[-4:] == ["runtimes", "1", "finite", "True"], out.stdout
