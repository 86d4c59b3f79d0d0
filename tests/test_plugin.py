"""The plugin entry point and the graph-safe custom ops (CPU: import
discipline, idempotence, fake-tensor shapes; GPU: the ops equal the direct
kernel calls bit for bit)."""
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from _util import bits_of, pkg

ROOT = Path(__file__).resolve().parent.parent


def test_plugin_import_is_stdlib_only():
    code = (
        "import sys, importlib.util\n"
        f"sys.path.insert(0, {str(ROOT)!r})\n"
        "import __graft_entry__ as g\n"
        "spec = importlib.util.spec_from_file_location('p', g.PKG_DIR / 'plugin' / '__init__.py')\n"
        "m = importlib.util.module_from_spec(spec); spec.loader.exec_module(m)\n"
        "bad = [n for n in ('torch', 'numpy', 'vllm') if n in sys.modules]\n"
        "print(','.join(bad))\n")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True)
    assert out.stdout.strip() == "", f"plugin import pulled in {out.stdout.strip()}"


def test_register_is_idempotent():
    plugin = pkg("plugin")
    a = plugin.register()
    b = plugin.register()
    assert a is b
    assert a["ops"] == "smx"
    import torch
    assert hasattr(torch.ops.smx, "q4_0_gemv")


def test_fake_shapes():
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode
    pkg("plugin").register()
    with FakeTensorMode():
        x = torch.empty((1, 2560), dtype=torch.bfloat16)
        w = torch.empty((9728, 1440), dtype=torch.uint8)
        assert torch.ops.smx.q4_0_gemv(x, w, 9728, 2560).shape == (1, 9728)
        assert torch.ops.smx.q4_0_gemv_swiglu(x, w, 4864, 2560).shape == (1, 4864)
        lut = torch.empty(4096, dtype=torch.bfloat16)
        assert torch.ops.smx.q4_0_gemv_gelu(x, w, lut, 4864, 2560).shape == (1, 4864)
        y, r = torch.ops.smx.add_rmsnorm(x, x, torch.empty(2560, dtype=torch.bfloat16), 1e-6)
        assert y.shape == r.shape == (1, 2560)
        q = torch.empty((1, 32, 128), dtype=torch.bfloat16)
        kc = torch.empty((4, 128, 8, 128), dtype=torch.bfloat16)
        out = torch.ops.smx.splitkv_decode_attention(
            q, kc, kc, torch.empty((1, 4), dtype=torch.int32), torch.empty(1, dtype=torch.int32),
            4, 0.088)
        assert out.shape == (1, 32, 128)
        ids = torch.ops.smx.argmax(torch.empty((3, 1000), dtype=torch.bfloat16))
        assert ids.shape == (3,) and ids.dtype == torch.int64
        # the reference's per-layer seam: (y, residual) shaped like its inputs
        # (src/spark_vllm_ascend/integration/model.py:81-82)
        y, r = torch.ops.smx.layer_run(x, x, torch.empty(1, dtype=torch.int64),
                                       "model.layers.0.self_attn.attn")
        assert y.shape == r.shape == (1, 2560) and y.dtype == r.dtype == torch.bfloat16


@pytest.mark.gpu
def test_custom_ops_match_direct_calls():
    import torch
    pkg("plugin").register()
    ops = pkg("native.torch_ops")
    w_mod = pkg("integration.weights")
    dev = torch.device("cuda:0")
    w = w_mod.synthetic_q4_0(1024, 2560, 3, dev)
    x = torch.randn((1, 2560), device=dev).to(torch.bfloat16)
    np.testing.assert_array_equal(bits_of(torch.ops.smx.q4_0_gemv(x, w, 1024, 2560)),
                                  bits_of(ops.q4_0_gemv(x, w, 1024, 2560)))
    np.testing.assert_array_equal(bits_of(torch.ops.smx.q4_0_gemv_swiglu(x, w, 512, 2560)),
                                  bits_of(ops.q4_0_gemv_swiglu(x, w, 512, 2560)))
    lut = ops.gelu_table(dev)
    np.testing.assert_array_equal(bits_of(torch.ops.smx.q4_0_gemv_gelu(x, w, lut, 512, 2560)),
                                  bits_of(ops.q4_0_gemv_gelu(x, w, lut, 512, 2560)))
    logits = torch.randn((2, 5000), device=dev).to(torch.bfloat16).float().cpu()
    ids = torch.ops.smx.argmax(logits.to(torch.bfloat16).to(dev)).cpu()
    for r in range(2):  # the first index holding the row maximum
        top = logits[r].max()
        assert logits[r, ids[r]] == top and not (logits[r, :ids[r]] == top).any()
