"""The C-ABI library loads, exports every symbol include/gemmaembed.h declares, and its binding's
signatures cover exactly that set. No compute calls: these run without a GPU."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gemmaembed.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(re.findall(r"\b(ge_[a-z0-9_]+)\s*\(", text))
    # typedef'd function pointer types are not symbols
    names -= set(re.findall(r"\(\s*\*\s*(ge_[a-z0-9_]+)\s*\)", text))
    return names


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ("ge_create", "ge_destroy", "ge_upload_model", "ge_forward", "ge_forward_trace", "ge_last_error",
              "ge_op_gemm_q8", "ge_op_attention", "ge_model_load", "ge_model_embed", "ge_plan_batches"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import gemma_embed as ge
    lib = ctypes.CDLL(ge.LIB_PATH)
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_signatures_match_header():
    import gemma_embed as ge
    assert set(ge.SIGNATURES) == declared_functions()


def test_oracle_library_loads():
    import ge_oracle as ora
    assert ora.lib.ora_gelu_tanh(0.0) == 0.0


def test_library_links_no_torch():
    import gemma_embed as ge
    with open(ge.LIB_PATH, "rb") as f:
        blob = f.read()
    assert b"libtorch" not in blob and b"libc10" not in blob


def test_create_without_gpu_reports_an_error():
    import gemma_embed as ge
    if os.environ.get("GE_EXPECT_GPU"):
        pytest.skip("a GPU is present")
    try:
        ctx = ge.Context.create(0)
    except ge.GemmaEmbedError as e:
        assert e.code in (1, 4, 8) and e.message
    else:  # a GPU is visible after all
        ctx.close()
