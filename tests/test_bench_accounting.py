"""The bench line's roofline arithmetic, pinned on the CPU against figures worked out by hand from
the config-2 and config-5 shapes rather than from bench.py's own formulas: 8,454,144 linear FLOPs
per token and layer (q/k/v, o, gate/up, down of the 768-wide text model), 4.9013e11 attention FLOPs
for 32 texts of 512 tokens at half window 256 with five sliding layers to one global, 1.2147e13
FLOPs per config-5 batch, the gate/up launch's 66.45 MB of algorithmic bytes, and the traffic
figure the committed counter profile states."""
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_module", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_config2_linear_flops_per_token_and_layer():
    b = _bench()
    per_layer = sum(b.gemm_flops(1).values())
    # q, k, v (3 + 2 heads of 256 from 768) + o (768 from 768) + gate/up (2 x 1152) + down (768 from 1152)
    assert per_layer == 2 * (1280 * 768 + 768 * 768 + 2304 * 768 + 768 * 1152) == 8_454_144


def test_config2_attention_flops():
    b = _bench()
    got = b.attention_flops([512] * 32)
    assert abs(got - 4.9013e11) / 4.9013e11 < 1e-4
    # a global layer sees every pair of a 512-token text: 4 hd H n^2 per text
    assert b.attention_flops([512], pattern=(0,)) == 4 * 256 * 3 * 512 * 512


def test_config5_flops():
    b = _bench()
    gemm, attn = b.vision_flops()
    assert abs((gemm + attn) - 1.2147e13) / 1.2147e13 < 1e-4
    assert attn == 16 * 8 * 4 * 72 * 16 * 2304 * 2304


def test_gate_up_algorithmic_bytes_and_profiled_traffic():
    b = _bench()
    assert b.gemm_bytes(16384)["gemm_gate_up"] == 2 * 16384 * 768 + 2 * 2304 * 768 + 2 * 16384 * 1152  # 66.45 MB
    traffic, kernel = b.measured_traffic("gemm_gate_up")
    assert kernel == "ge::gemm_kernel<ge::GemmCfg<128, 256, 2, 4, 32, 3>, 2>"
    # the profile's FETCH_SIZE and WRITE_SIZE totals, scaled: more than the algorithmic bytes (X row
    # blocks re-read by every column tile), writes exactly the 37.75 MB GeGLU product
    assert 66_453_504 < traffic < 4 * 66_453_504
