import os
import sys
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("gemma-embed-swift_amd", "oracle", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C-ABI library")


@pytest.fixture(scope="session")
def model_dir():
    d = tempfile.mkdtemp(prefix="ge_models_")
    yield d


@pytest.fixture(scope="session")
def tiny_gguf(model_dir):
    import gemma_embed as ge
    return ge.synth_write_gguf(os.path.join(model_dir, "tiny.gguf"), **ge.TINY)


@pytest.fixture(scope="session")
def config2_gguf(model_dir):
    import gemma_embed as ge
    return ge.synth_write_gguf(os.path.join(model_dir, "config2.gguf"), **ge.CONFIG2)


@pytest.fixture(scope="session")
def tiny_vision_gguf(model_dir):
    import gemma_embed as ge
    return ge.synth_write_vision_gguf(os.path.join(model_dir, "tiny_vision.gguf"), **ge.TINY_VISION)


@pytest.fixture(scope="session")
def config5_vision_gguf(model_dir):
    import gemma_embed as ge
    return ge.synth_write_vision_gguf(os.path.join(model_dir, "config5_vision.gguf"), **ge.CONFIG5_VISION)


@pytest.fixture(scope="session")
def tiny_ple_gguf(model_dir):
    import gemma_embed as ge
    return ge.synth_write_gguf(os.path.join(model_dir, "tiny_ple.gguf"), **ge.TINY_PLE)


@pytest.fixture(scope="session")
def real_shapes_gguf(model_dir):
    import gemma_embed as ge
    return ge.synth_write_gguf(os.path.join(model_dir, "real_shapes.gguf"), **ge.REAL_SHAPES)
