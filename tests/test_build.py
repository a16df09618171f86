"""The build's kernel-resource gate: the compiler's per-kernel
resource-usage remarks are parsed, and a kernel with VGPR spills or a
scratch segment fails the build (SGPR spills, which land in VGPR lanes, pass).
"""
import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build_mod():
    path = os.path.join(ROOT, "apus-glm5.3-flash_amd", "build.py")
    spec = importlib.util.spec_from_file_location("apus_build", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _remarks(name, scratch, sgpr, vgpr):
    f = "k.hip:10:1: remark: "
    tag = " [-Rpass-analysis=kernel-resource-usage]"
    return "\n".join([
        f + "Function Name: " + name + tag,
        f + "    VGPRs: 128" + tag,
        f + "    ScratchSize [bytes/lane]: %d" % scratch + tag,
        f + "    SGPRs Spill: %d" % sgpr + tag,
        f + "    VGPRs Spill: %d" % vgpr + tag,
        "   10 | __global__ void k() {",
        "      | ^",
    ])


def test_resource_remarks_parsed_and_context_dropped():
    b = _build_mod()
    text = "\n".join([_remarks("_Z1av", 0, 5, 0), "real warning line",
                      _remarks("_Z1bv", 28, 0, 6)])
    usage, rest = b.resource_usage(text)
    assert usage == {"_Z1av": {"scratch": 0, "sgpr_spill": 5, "vgpr_spill": 0},
                     "_Z1bv": {"scratch": 28, "sgpr_spill": 0, "vgpr_spill": 6}}
    assert rest == "real warning line"


def test_spilling_kernel_fails_the_gate():
    b = _build_mod()
    ok, _ = b.resource_usage(_remarks("_Z1av", 0, 32, 0))
    b.check_resources(ok, required=())         # SGPR spills alone pass
    for scratch, vgpr in ((0, 1), (4, 0)):
        bad, _ = b.resource_usage(_remarks("_Z1bv", scratch, 0, vgpr))
        with pytest.raises(RuntimeError, match="_Z1bv"):
            b.check_resources(bad, required=())


def test_gate_fails_without_remarks():
    """No parsed remarks, a required kernel without remarks, or a remark
    block without its spill and scratch figures fail the build: a gate that
    saw nothing must not pass."""
    b = _build_mod()
    with pytest.raises(RuntimeError, match="no kernel-resource-usage"):
        b.check_resources({})
    ok, _ = b.resource_usage(_remarks("_Z12k_moe_decodev", 0, 0, 0))
    b.check_resources(ok, required=("k_moe_decode",))
    with pytest.raises(RuntimeError, match="k_pf_gemm"):
        b.check_resources(ok, required=("k_moe_decode", "k_pf_gemm"))
    with pytest.raises(RuntimeError, match="without spill"):
        b.check_resources({"_Z1cv": {"scratch": 0}}, required=())
