"""CPU bounds audit of every kernel launch of the text forward (tests/launch_audit.py): for each
synthetic model the GPU tests and the bench load and each pack shape they run, no access of any
launch leaves its allocation. The planted-mistake cases check that the audit notices a workspace
one row short, a V^T buffer one row short, slack-free legacy attention and the split forward's
attention given plain row offsets instead of its part bases."""
import numpy as np
import pytest

import gemma_embed as ge
import launch_audit as la

MODELS = {"tiny": ge.TINY, "tiny_ple": ge.TINY_PLE, "config2": ge.CONFIG2, "outlier_norms": ge.OUTLIER_NORMS,
          "real_shapes": ge.REAL_SHAPES,
          # config 2 loaded with split-precision scores on every layer (ge_load_options.split_scores)
          "config2_split_scores": dict(ge.CONFIG2, split_scores=True)}

SHORT = [[1], [2], [40, 9], [63], [64], [65], [1] * 64, [5, 0, 7], [300], [1, 65], [100, 33, 7, 1]]
LONG = [[1024] * 8, [512] * 32, [8192], [8192, 8192], [4096, 1], [1, 4096], [2048] * 8, [3000, 5000, 192],
        [7] * 600 + [4000]]


def config3_batches():
    """BASELINE config 3's 256 ragged texts (lengths U[8, 256]) planned into batches of at most
    8192 tokens, as the bench packs them."""
    lengths = [int(n) for n in ge.synth_tokens(31, 8, 257, 256)]
    return [[lengths[i] for i in r] for r in ge.plan_batches(lengths, [8192])]


def cases():
    out = []
    for name in MODELS:
        packs = SHORT + (LONG + config3_batches() if name in ("config2", "real_shapes", "config2_split_scores") else [[1024] * 8, [8192]])
        out += [(name, p) for p in packs]
    return out


@pytest.mark.parametrize("name,lengths", cases(), ids=lambda v: v if isinstance(v, str) else f"{len(v)}x{max(v)}")
def test_every_access_inside_its_allocation(name, lengths):
    m = la.model_of(MODELS[name])
    b = la.plan(m, lengths)
    a = la.replay(m, b)
    assert not a.errors, "\n".join(a.errors[:10])
    assert a.checked > 20 * m["layers"]
    assert not la.check_parts_disjoint(m, b)


def test_tokens_outside_every_sequence():
    # rows between sequences (unused packing gaps) take the last V^T slack column
    m = la.model_of(ge.CONFIG2)
    b = la.plan(m, [10, 20, 0, 33], gaps=[3, 5, 1, 7])
    assert b["vcol"].max() == b["vt_cols"] - 1
    a = la.replay(m, b)
    assert not a.errors, "\n".join(a.errors[:10])


def test_split_plans_cover_all_work():
    for lengths in ([512] * 32, [1024] * 8, [7] * 600 + [4000], [3000, 5000, 192]):
        m = la.model_of(ge.CONFIG2)
        b = la.plan(m, lengths)
        assert b["n_parts"] > 1
        assert b["part_work"][-1] == len(b["work2"])
        for p in range(b["n_parts"]):
            w = b["work2"][b["part_work"][p]:b["part_work"][p + 1]]
            assert np.all(w[:, 0] >= b["part_row"][p]) and np.all(w[:, 0] + w[:, 1] <= b["part_row"][p + 1])


# ---- planted mistakes: each must be reported

def test_audit_reports_a_workspace_one_row_short(monkeypatch):
    m = la.model_of(ge.CONFIG2)
    b = la.plan(m, [40, 9])
    real = la.workspace

    def short(m_, b_):
        ws = real(m_, b_)
        R = (b_["n"] + 63) // 64 * 64 + la.ROW_SLACK
        ws["x"] = ws["x"] // R * (b_["n"] - 1)
        return ws

    monkeypatch.setattr(la, "workspace", short)
    a = la.replay(m, b)
    assert any(e.startswith("embed_norm: x") for e in a.errors)
    assert any(e.startswith("residual_norm: x") for e in a.errors)


def test_audit_reports_a_vt_buffer_one_row_short(monkeypatch):
    m = la.model_of(ge.CONFIG2)
    b = la.plan(m, [1024] * 8)
    real = la.workspace

    def short(m_, b_):
        ws = real(m_, b_)
        ws["vt"] -= b_["vt_cap"] * la.F16
        return ws

    monkeypatch.setattr(la, "workspace", short)
    a = la.replay(m, b)
    assert any(e.startswith("attention: vt") for e in a.errors)
    assert any(e.startswith("gemm_qkv: vt") for e in a.errors)


def test_audit_reports_legacy_attention_without_row_slack(monkeypatch):
    # hd 256 with 4 query heads per KV head takes the legacy kernel, whose 64-key blocks read past
    # the sequence's end: a pack [1, 65] reads row 128 of a 66-token batch
    spec = dict(ge.TINY, heads=4, kv_heads_swa=1, kv_heads_global=1, head_dim_swa=256, head_dim_global=256)
    m = la.model_of(spec)
    assert not m["layer"][0]["attn_v2"]
    b = la.plan(m, [1, 65])
    assert not la.replay(m, b).errors
    monkeypatch.setattr(la, "ROW_SLACK", 0)
    a = la.replay(m, b)
    assert any(e.startswith("attention: k") for e in a.errors)


def test_audit_reports_split_attention_without_part_bases(monkeypatch):
    m = la.model_of(ge.CONFIG2)
    b = la.plan(m, [512] * 32)
    real = la.attention_items

    def absolute(a, kernel, work, H, KV, HD, q, k, vt, vt_cols, o, item_queries, q_lo=None, k_lo=None):
        # the part's row offset added on top of the absolute row indices the work items hold
        r0 = int(work[:, 0].min())
        q, k, o = (q[0], r0 * H * HD * la.F16), (k[0], r0 * KV * HD * la.F16), (o[0], r0 * H * HD * la.F16)
        return real(a, kernel, work, H, KV, HD, q, k, vt, vt_cols, o, item_queries, q_lo, k_lo)

    monkeypatch.setattr(la, "attention_items", absolute)
    a = la.replay(m, b)
    assert any(e.startswith("attention: q") for e in a.errors)


def test_audit_reports_empty_work_items_without_the_early_exit():
    # a work list that reached the kernels as zeros (seq_len 0): without the kernels' len <= 0 exit
    # the (len - 1) in the resource ranges wraps to about 4 GB
    m = la.model_of(ge.CONFIG2)
    b = la.plan(m, [512] * 4)
    a = la.Audit(la.workspace(m, b))
    zeros = np.zeros_like(b["work2"])
    la.attention_items(a, "attention", zeros, 3, 1, 256, ("q", 0), ("k", 0), ("vt", 0), b["vt_cap"], ("attn", 0), 64)
    assert not a.errors
    la.attention_items(a, "attention", zeros, 3, 1, 256, ("q", 0), ("k", 0), ("vt", 0), b["vt_cap"], ("attn", 0), 64,
                       leave_empty=False)
    assert any("does not fit 32 bits" in e or "outside" in e for e in a.errors)
