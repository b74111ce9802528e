"""CPU tests of the C ABI library (no GPU needed): it loads, exports every
function declared in include/gptoss_moe.h, and rejects bad arguments with a
status code and a message instead of aborting (the reference aborts,
include/cuda_utils.h:17-35).  None of these calls reaches a kernel launch."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gptoss_moe.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gptoss_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def g():
    import gptoss_moe
    return gptoss_moe


def test_exports_every_declared_symbol(g):
    names = declared_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(g.lib, n)]
    assert not missing, missing


def test_abi_version_and_defaults(g):
    assert g.lib.gptoss_abi_version() == 7
    cfg = g.default_config(128, 64)
    assert (cfg.hidden_size, cfg.num_experts, cfg.top_k, cfg.intermediate_size) == (2880, 128, 4, 2880)
    assert abs(cfg.swiglu_alpha - 1.702) < 1e-6 and cfg.swiglu_limit == 7.0
    assert cfg.prefill_min_tokens == 128  # decode batches (<= 64) stream the weights
    assert cfg.decode_exact == 0          # decode on the matrix cores unless asked for the exact kernels
    assert g.lib.gptoss_moe_config_default(None, 128, 1) == g.GPTOSS_ERR_INVALID
    assert b"NULL" in g.lib.gptoss_last_error()


def test_tiled_size_and_shape_errors(g):
    nb, sb = g.tiled_size(5760, 2880)
    assert nb == 5760 * 1440                     # nibbles are only permuted
    # 15 scales per (tile, part, row) padded to 16, then one per (row, block) in slot order
    assert sb == 90 * 6 * 64 * 16 + 5760 * 90
    nb, sb = g.tiled_size(2880, 2880)
    assert nb == 2880 * 1440 and sb == 45 * 6 * 64 * 16 + 2880 * 90
    with pytest.raises(ValueError):
        g.tiled_size(64, 33)                     # K not a multiple of the MXFP4 block
    with pytest.raises(g.GptossError) as e:
        g.tiled_size(63, 64)
    assert e.value.code == g.GPTOSS_ERR_UNSUPPORTED


def test_layer_state_errors(g):
    L = g.MoELayer()
    with pytest.raises(g.GptossError) as e:
        L.forward_prenormed(_FakeT(1), None, out=_FakeT(1))
    assert e.value.code == g.GPTOSS_ERR_STATE
    cfg = g.default_config(128, 8)
    cfg.top_k = 3
    with pytest.raises(ValueError, match="top_k"):
        L.init(cfg, 0, router_weight=_FakeT(1), mlp1=([], []), mlp2=([], []))
    cfg = g.default_config(300, 8)
    with pytest.raises(g.GptossError) as e:
        L.init(cfg, 0, router_weight=_FakeT(1), mlp1=([], []), mlp2=([], []))
    assert e.value.code == g.GPTOSS_ERR_UNSUPPORTED
    cfg = g.default_config(128, 0)
    with pytest.raises(ValueError, match="max_tokens"):
        L.init(cfg, 0, router_weight=_FakeT(1), mlp1=([], []), mlp2=([], []))
    cfg = g.default_config(128, 8)
    with pytest.raises(ValueError, match="router_weight"):
        L.init(cfg, 0, router_weight=None, mlp1=([], []), mlp2=([], []))
    with pytest.raises(ValueError, match="aligned"):
        L.init(cfg, 0, router_weight=_FakeT(2), mlp1=([], []), mlp2=([], []))
    L.destroy()


def test_layer_forward_argument_checks(g):
    """The Python layer refuses tensors the kernels would misread before
    anything reaches the library: wrong width, dtype, rank, a transposed
    view, another device, mismatched rows, and routing tensors of the wrong
    dtype or shape.  The layer is given a config without init (no GPU), so
    every call here must fail in the host-side checks."""
    import torch
    L = g.MoELayer()
    L.cfg, L.device = g.default_config(128, 8), 0
    H = L.cfg.hidden_size

    def bf(*shape):
        return torch.zeros(shape, dtype=torch.bfloat16)

    cases = [
        (lambda: L.forward_prenormed(bf(2, H - 64)), "shape"),               # hidden width below H
        (lambda: L.forward_prenormed(torch.zeros(2, H)), "dtype"),           # fp32 activations
        (lambda: L.forward_prenormed(bf(2, 1, H)), "2-D"),
        (lambda: L.forward_prenormed(bf(H, 2).t()), "contiguous"),            # transposed view
        (lambda: L.forward_prenormed(bf(2, H)), "cuda:0"),                    # host tensor
        (lambda: L.forward(bf(2, H)), "cuda:0"),
        (lambda: L.forward_residual(bf(2, H), bf(2, H)), "cuda:0"),
        (lambda: g._check_tensor("delta", bf(3, H), 0, 2, H, 2, g._BF16), "delta has shape"),  # rows != T
        (lambda: L.forward_routed(bf(2, H), torch.zeros(2, 4, dtype=torch.int64),
                                  torch.zeros(2, 4)), "cuda:0|dtype"),
    ]
    for call, msg in cases:
        with pytest.raises(ValueError, match=msg):
            call()
    # the routing tensors' own rules, on the helper the layer calls
    with pytest.raises(ValueError, match="expert_indices has dtype"):
        g._check_tensor("expert_indices", torch.zeros(2, 4, dtype=torch.int64), 0, 4, 4, 2, (torch.int32,))
    with pytest.raises(ValueError, match="expert_weights has shape"):
        g._check_tensor("expert_weights", torch.zeros(2, 8), 0, 4, 4, 2, (torch.float32,))
    L.cfg = None
    L.destroy()


def test_stage_argument_errors(g):
    lib = g.lib
    assert lib.gptoss_moe_route(None, None, None, 0, 128, 2880, 4, 0, None, None, None, None, None) == g.GPTOSS_OK
    assert lib.gptoss_moe_route(None, None, None, 4, 128, 2880, 3, 0, None, None, None, None, None) == \
        g.GPTOSS_ERR_INVALID
    assert b"top_k" in lib.gptoss_last_error()
    assert lib.gptoss_moe_route(None, None, None, 4, 128, 2881, 4, 0, None, None, None, None, None) == \
        g.GPTOSS_ERR_INVALID
    assert lib.gptoss_topk_softmax_forward(None, 0, None, None, None, 4, 128, 9, None) == g.GPTOSS_ERR_INVALID
    assert lib.gptoss_moe_permute_plan(None, 4, 4, 999, None, None, None, None, None, None, None) == \
        g.GPTOSS_ERR_UNSUPPORTED
    assert lib.gptoss_mxfp4_gemv_forward(None, 1, None, None, None, None, 64, 48, None) == g.GPTOSS_ERR_INVALID
    assert lib.gptoss_swiglu_forward(None, None, -1, 4, 1.702, 7.0, None) == g.GPTOSS_ERR_INVALID
    assert lib.gptoss_moe_combine_forward(None, None, None, None, None, 2, 64, 9, None) == g.GPTOSS_ERR_INVALID
    assert lib.gptoss_mxfp4_dequant(None, None, 64, 64, None, None) == g.GPTOSS_ERR_INVALID
    assert lib.gptoss_moe_route_scratch_bytes(4096, 128, 4) >= 1  # reserved: a non-empty allocation


class _FakeT:
    """Stand-in with a data_ptr() for argument-validation tests (never dereferenced)."""

    def __init__(self, addr):
        self._a = addr * 4096 + (0 if addr % 2 else 8)

    def data_ptr(self):
        return self._a

    @property
    def shape(self):
        return (1, 2880)


# The reference's C++ operator interface as its callers declare it
# (engine.cu:175-196, transformer.cu:106-121; defined at moe_layer.cu:1556-1615),
# written out as demangled signatures.
REFERENCE_OPERATOR_SIGNATURES = {
    "gptoss::moe_layer_create()",
    "gptoss::moe_layer_destroy(gptoss::MoELayer*)",
    "gptoss::moe_layer_forward(gptoss::MoELayer*, __hip_bfloat16 const*, __hip_bfloat16*, int, ihipStream_t*)",
    "gptoss::moe_layer_forward_prenormed(gptoss::MoELayer*, __hip_bfloat16 const*, __hip_bfloat16 const*, "
    "__hip_bfloat16*, int, ihipStream_t*)",
    "gptoss::moe_layer_get_ffn_norm_weight(gptoss::MoELayer*)",
    "gptoss::moe_layer_init(gptoss::MoELayer*, int, int, int, gptoss::EPComm*, gptoss::CublasHandle const*, "
    "gptoss::CublasHandle const*, ihipStream_t*, ihipStream_t*, __hip_bfloat16 const*, __hip_bfloat16 const*, "
    "__hip_bfloat16 const*, __hip_bfloat16 const*, __hip_bfloat16 const*, gptoss::MXFP4Weight*, "
    "gptoss::MXFP4Weight*, " + ", ".join(
        ["__hip_bfloat16*", "__hip_bfloat16*", "int*", "float*", "int*", "__hip_bfloat16*", "int*", "int*", "int*",
         "int*"] + ["__hip_bfloat16*"] * 9) + ", ncclComm*)",
}


def test_cpp_operator_shim_exports_reference_signatures():
    """libgptoss_moe_compat.so exports the reference's gptoss::moe_layer_*
    with identical signatures (so identical mangled names for its callers)."""
    import shutil
    import subprocess
    lib = os.path.join(ROOT, "hip-kernels_amd", "libgptoss_moe_compat.so")
    assert os.path.exists(lib), "build the library first (make -C hip-kernels_amd)"
    if shutil.which("nm") is None or shutil.which("c++filt") is None:
        pytest.skip("binutils nm/c++filt not available")
    names = subprocess.run(["nm", "-D", "--defined-only", lib], check=True, capture_output=True, text=True).stdout
    mangled = [ln.split()[-1] for ln in names.splitlines() if "gptoss" in ln]
    demangled = set(subprocess.run(["c++filt"], input="\n".join(mangled), check=True, capture_output=True,
                                   text=True).stdout.split("\n")) - {""}
    missing = REFERENCE_OPERATOR_SIGNATURES - demangled
    assert not missing, missing


def test_bench_rejects_several_gpus():
    """bench.py measures one GPU: --gpus above 1 exits with status 2 and says so."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "one GPU only" in r.stderr and r.stdout == ""


def test_binding_fails_loudly_without_library(tmp_path, monkeypatch):
    """The Python binding has no CPU fallback: imported from a directory that
    holds no built libgptoss_moe.so, it raises ImportError naming the library."""
    import importlib.util
    import shutil
    monkeypatch.delenv("GPTOSS_MOE_LIB", raising=False)
    src = os.path.join(ROOT, "hip-kernels_amd", "gptoss_moe.py")
    shutil.copy(src, tmp_path / "gptoss_moe_nolib.py")
    spec = importlib.util.spec_from_file_location("gptoss_moe_nolib", tmp_path / "gptoss_moe_nolib.py")
    mod = importlib.util.module_from_spec(spec)
    with pytest.raises(ImportError, match="libgptoss_moe.so is not built"):
        spec.loader.exec_module(mod)
