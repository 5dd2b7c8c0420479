"""The C ABI library without a GPU: it loads, exports every symbol the header
declares (with the ctypes binding covering each), and its host-only entry
points validate arguments and report errors instead of crashing."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qppocr_hip.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"QPH_API\s+[\w\s\*]+?\b(qph_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from qppocr_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from qppocr_amd import build
        build.build()
    return _lib.load()


def test_header_declares_the_operator_set():
    syms = declared_symbols()
    for s in ["qph_conv2d", "qph_sgemm", "qph_softmax_last_dim", "qph_layernorm", "qph_attention",
              "qph_ctc_argmax", "qph_convtranspose2d", "qph_net_create", "qph_net_run"]:
        assert s in syms
    assert len(syms) >= 30


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    from qppocr_amd import _lib
    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_conv2d_out_shape_host_only(lib):
    from qppocr_amd import _lib, ops
    p = ops.conv_params(2, 2, 1, 1)
    assert ops.conv2d_out_shape((1, 3, 640, 640), (16, 3, 3, 3), p) == (1, 16, 320, 320)
    p = ops.conv_params(3, 1, 0, 1)
    assert ops.conv2d_out_shape((32, 256, 3, 40), (256, 1, 3, 3), ops.conv_params(3, 1, 0, 1, group=256)) == (32, 256, 1, 40)
    # end padding larger than begin padding (kernels.rs:594-635)
    assert ops.conv2d_out_shape((1, 4, 1, 1), (4, 1, 3, 3),
                                _lib.ConvParams(1, 1, 0, 0, 2, 2, 1, 1, 4)) == (1, 4, 1, 1)
    with pytest.raises(_lib.QphError) as e:
        ops.conv2d_out_shape((1, 3, 8, 8), (16, 2, 3, 3), ops.conv_params())
    assert e.value.code == -1 and "group" in str(e.value)
    with pytest.raises(_lib.QphError) as e:
        ops.conv2d_out_shape((1, 3, 8, 8), (16, 3, 3, 3), _lib.ConvParams(1, 1, 0, 0, 0, 0, 2, 2, 1))
    assert e.value.code == -3                         # dilation unsupported
    with pytest.raises(_lib.QphError):
        ops.conv2d_out_shape((1, 3, 2, 2), (16, 3, 5, 5), ops.conv_params())   # empty output


def test_null_context_is_an_error_not_a_crash(lib):
    P = ctypes.c_void_p
    assert lib.qph_sync(None) == -1
    assert b"null context" in lib.qph_last_error()
    act = None
    assert lib.qph_conv2d(None, None, None, None, None, None, None, act, None, None, None) == -1
    assert lib.qph_softmax_last_dim(None, None, 1, 1) == -1
    assert lib.qph_pack_crops(None, 1, None, None, None, None, 48, 320, None) == -1
    assert lib.qph_plan_run(None, None, 1, None) == -1
    assert lib.qph_net_run(None, None, 0, None) == -1
    assert lib.qph_net_set_real_n(None, 1) == -1
    assert lib.qph_net_real_n(None, None, None) == -1
    assert lib.qph_net_destroy(None) == 0
    assert lib.qph_ctx_destroy(None) == 0
    out = P()
    assert lib.qph_ctx_create(0, None) == -1


def test_ctx_create_without_gpu_reports_error(lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    out = ctypes.c_void_p()
    rc = lib.qph_ctx_create(0, ctypes.byref(out))
    assert rc != 0 and out.value is None
    assert lib.qph_last_error() != b""


def test_ops_refuse_host_tensors(lib):
    import torch
    from qppocr_amd import ops
    with pytest.raises((ValueError, RuntimeError)):
        ops.softmax_last_dim(torch.zeros(4, 8), 8)


def test_version(lib):
    assert b"gfx950" in lib.qph_version()



def _spec_with_outputs(outputs):
    """A two-tensor ACT graph spec (no weights) with the given output ids."""
    from qppocr_amd import nets
    g = nets.Graph((1, 4, 2, 2))
    t = g.tensor((1, 4, 2, 2))
    g.nodes.append(dict(op=nets.OP_ACT, inp=0, in2=-1, out=t, out2=-1, w=-1, bias=-1, w2=-1,
                        ws=(0, 0, 0, 0), w2s=(0, 0, 0, 0), cp=(1,) * 9, act=2, res_up=0,
                        trans_out=0, y_ctotal=0, y_coff=0, y_up=1, heads=0, dh=0, eps=0.0,
                        scale=0.0))
    g.outputs = list(outputs)
    return g.to_c()


def test_net_create_checks_the_spec_before_the_device(lib):
    """Output ids outside the tensor table are refused before any device
    work (a bad id would otherwise index host tables out of range)."""
    for bad in ([2], [-1], [0, 7]):
        spec, keep = _spec_with_outputs(bad)
        out = ctypes.c_void_p()
        rc = lib.qph_net_create(None, ctypes.byref(spec), None, ctypes.byref(out))
        assert rc == -1 and b"output" in lib.qph_last_error(), bad
        assert out.value is None
    spec, keep = _spec_with_outputs([1])
    spec.n_outputs = 1
    spec.outputs = None
    assert lib.qph_net_create(None, ctypes.byref(spec), None, ctypes.byref(ctypes.c_void_p())) == -1
    assert b"output list" in lib.qph_last_error()
    # a valid spec gets as far as the context check
    spec, keep = _spec_with_outputs([1])
    assert lib.qph_net_create(None, ctypes.byref(spec), None, ctypes.byref(ctypes.c_void_p())) == -1
    assert b"NULL context" in lib.qph_last_error()
