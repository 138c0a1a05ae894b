"""Bounds audit of the text forward's kernel launches, replayed on the CPU (test infrastructure).

For every kernel the forward launches, this module restates the index arithmetic by which the
kernel's threads address global memory, the workspace the runtime allocates for a batch
(ensure_workspace_impl, csrc/device/runtime.cpp:617), the batch plan it stages (plan_batch :724,
vt_layout :703, stage :837) and the launch sequence with its pointer arguments (encode :915 for one
stream, encode_split :1051 for a batch split over streams, both ending in encode_tail :904). Every access range of every launch is
checked against the allocation its pointer falls in.

- Plain loads and stores: the range of element indices the kernel's guards let through.
- Buffer-resource reads (the GEMM and attention copies, `buffer_rsrc` in csrc/device/common.hpp):
  the hardware returns zeros for offsets past a resource's size, so what must hold is that the
  resource's whole range lies inside the allocation and its size fits the 32-bit field.
- LDS is not covered: an LDS access outside the workgroup's allocation does not fault.

Sizes are in bytes; a pointer is (buffer name, byte offset)."""
import numpy as np

F32, F16, I32 = 4, 2, 4
ROW_SLACK = 256          # kRowSlack, csrc/device/kernels.hpp:29
ATTN_QUERIES = 32        # kAttnQueries, kernels.hpp:26
ATTN_QUERIES_V2 = 64     # kAttnQueriesV2, kernels.hpp:139
SMALL_ITEMS = 256        # kAttnSmallItems, runtime.cpp
SPLIT_MIN_TOKENS = 4096  # kSplitMinTokens, runtime_internal.hpp
MAX_PARTS = 4            # kMaxParts, runtime_internal.hpp
SKINNY_MAX_ROWS = 512    # kSkinnyMaxRows, kernels.hpp
WORK_BYTES, SEQ_BYTES = 16, 8  # sizeof(AttnWork), sizeof(SeqRange)


# ---------------------------------------------------------------- model

def v2_supported(hd, H, KV):
    """attention_v2_supported (csrc/device/attention.hip:808)."""
    if hd == 512:
        return KV > 0 and H == 4 * KV
    if not (hd in (128, 256) and KV > 0 and H % KV == 0 and 1 <= H // KV <= 4):
        return False
    G = H // KV
    return 2 * G * 32 * hd * 2 + 2 * (2 * 32 * hd * 2) <= 160 * 1024


def model_of(spec):
    """The device model's shape and per-layer path flags, as upload() (runtime.cpp:450) derives them
    from a synthetic model spec (gemma_embed.synth_write_gguf's keyword arguments)."""
    H, D = spec["heads"], spec["hidden"]
    m = dict(layers=spec["layers"], hidden=D, heads=H, ff=spec["feed_forward"], out_dims=spec["out_dims"],
             pl=spec.get("per_layer_input", 0), vocab=spec["vocab"], window=spec["sliding_window"],
             max_tokens=min(spec.get("context_length", 8192) or 8192, 8192), layer=[])
    m.update(max_qd=0, max_kvd=0, max_qkv=0, max_kv_heads=0, any_precise=False, any_v2=False, all_v2=True,
             items32_ok=True)
    for i in range(m["layers"]):
        sliding = spec["pattern"][i] == 1
        hd = spec["head_dim_swa"] if sliding else spec["head_dim_global"]
        KV = spec["kv_heads_swa"] if sliding else spec["kv_heads_global"]
        sl = H + 2 * KV
        L = dict(sliding=sliding, hd=hd, kv=KV, qd=H * hd, kvd=KV * hd)
        # hd >= ge_ctx::split_head_dim (512, or 0 after ge_set_split_scores(ctx, 0)) and
        # attention_split_supported (attention.hip:1073)
        split_ok = (hd == 512 and H == 4 * KV) or (hd == 256 and H == 3 * KV)
        L["precise"] = split_ok and hd >= (0 if spec.get("split_scores") else 512)
        L["attn_v2"] = v2_supported(hd, H, KV)
        L["qkv_gn"] = hd in (128, 256) and sl in (3, 4, 5, 6, 8, 10) and KV * hd * 66 * 2 <= 64 * 1024
        L["qkv_fused"] = hd in (128, 256)
        if L["precise"]:
            L["qkv_gn"] = L["qkv_fused"] = False
        m["max_qd"] = max(m["max_qd"], L["qd"])
        m["max_kvd"] = max(m["max_kvd"], L["kvd"])
        m["max_kv_heads"] = max(m["max_kv_heads"], KV)
        m["max_qkv"] = max(m["max_qkv"], L["qd"] + 2 * L["kvd"])
        m["any_precise"] |= L["precise"]
        m["any_v2"] |= L["attn_v2"]
        m["all_v2"] &= L["attn_v2"]
        if L["attn_v2"] and H // KV > 3:
            m["items32_ok"] = False
        m["layer"].append(L)
    return m


# ---------------------------------------------------------------- batch plan and workspace

def plan(m, lengths, gaps=None):
    """plan_batch (runtime.cpp:724) for sequences of the given lengths packed back to back (with
    `gaps[i]` unused rows before sequence i): sequence ranges, both attention work lists as arrays
    of (seq_start, seq_len, q0, vt_start), the V^T layout (vt_layout :703) and the split into parts."""
    starts, r = [], 0
    for i, n in enumerate(lengths):
        r += gaps[i] if gaps else 0
        starts.append(r)
        r += n
    n_tok = r
    seqs = list(zip(starts, lengths))
    work = [(s, n, q0, 0) for s, n in seqs for q0 in range(0, n, ATTN_QUERIES)]
    b = dict(n=n_tok, seqs=seqs, work=np.array(work, dtype=np.int64).reshape(-1, 4), items=ATTN_QUERIES_V2,
             work2=np.zeros((0, 4), np.int64), vcol=None, vt_cols=0, n_parts=1, part_row=[0, n_tok],
             part_work=[0, 0])
    if m["any_v2"]:
        col, vstart = 0, []
        vcol = np.full(n_tok, -1, np.int64)
        for s, n in seqs:
            vstart.append(col)
            vcol[s:s + n] = col + np.arange(n)
            col += (n + 7) // 8 * 8
        cols = col + 64
        vcol[vcol < 0] = cols - 1
        b["vcol"], b["vt_cols"] = vcol, cols
        items64 = sum((n + ATTN_QUERIES_V2 - 1) // ATTN_QUERIES_V2 for _, n in seqs)
        if m["items32_ok"] and items64 * m["max_kv_heads"] < SMALL_ITEMS:
            b["items"] = 32
        w2 = [(s, n, q0, vs) for (s, n), vs in zip(seqs, vstart) for q0 in range(0, n, b["items"])]
        b["work2"] = np.array(w2, dtype=np.int64).reshape(-1, 4)
        b["part_work"] = [0, len(w2)]
    if m["all_v2"] and n_tok >= SPLIT_MIN_TOKENS and len(seqs) >= 2:
        cand = sorted(s for s, n in seqs if n and s > 0)
        cuts = []
        for p in range(1, MAX_PARTS):
            target = n_tok * p // MAX_PARTS
            best = -1
            for x in cand:
                if x > (cuts[-1] if cuts else 0) and (best < 0 or abs(x - target) < abs(best - target)):
                    best = x
            if 0 < best < n_tok:
                cuts.append(best)
        if cuts:
            rows = [0] + cuts + [n_tok]
            part = np.searchsorted(np.array(cuts), b["work2"][:, 0], side="right")
            order = np.argsort(part, kind="stable")
            counts = np.bincount(part, minlength=len(rows) - 1)
            if np.all(counts > 0):
                b["work2"] = b["work2"][order]
                b["n_parts"], b["part_row"] = len(rows) - 1, rows
                b["part_work"] = [0] + list(np.cumsum(counts))
    return b


def workspace(m, b):
    """Allocation sizes of ensure_workspace_impl (runtime.cpp:617) for a staged batch (a fresh
    context: every capacity is the batch's own)."""
    R = (b["n"] + 63) // 64 * 64 + ROW_SLACK
    D = m["hidden"]
    ws = dict(x=R * D * F32, h=R * D * F16, qkv=R * m["max_qkv"] * F32, q=R * m["max_qd"] * F16,
              k=R * m["max_kvd"] * F16, v=R * m["max_kvd"] * F16, attn=R * m["max_qd"] * F16, t=R * D * F32,
              act=R * m["ff"] * F16, out=R * m["out_dims"] * F32, hn=R * D * F32, tokens=R * I32, positions=R * I32,
              vcol=R * I32)
    if m["any_precise"]:
        ws.update(h3=R * 3 * D * F16, q_lo=R * m["max_qd"] * F16, k_lo=R * m["max_kvd"] * F16)
    if m["pl"] > 0:
        ws.update(ple=R * m["layers"] * m["pl"] * F32, ple_t=R * max(m["pl"], D) * F32, rs=R * F32, rs2=R * F32,
                  x16=R * D * F16, g16=R * m["pl"] * F16)
    seq_cap = max(len(b["seqs"]), 1)
    ws.update(seqs=seq_cap * SEQ_BYTES, pooled=seq_cap * m["out_dims"] * F32, pooled_n=seq_cap * D * F32,
              work=max(len(b["work"]), 1) * WORK_BYTES)
    if m["any_v2"]:
        ws["work2"] = max(len(b["work2"]), 1) * WORK_BYTES
        vt_cap = (b["vt_cols"] + 63) // 64 * 64
        ws["vt"] = m["max_kvd"] * vt_cap * F16
        b["vt_cap"] = vt_cap
    return ws


# ---------------------------------------------------------------- the checker

class Audit:
    def __init__(self, sizes):
        self.sizes = dict(sizes)
        self.errors = []
        self.checked = 0

    def span(self, kernel, ptr, lo, hi):
        """Bytes [lo, hi) past pointer ptr (scalars or arrays: the extreme values count)."""
        name, off = ptr
        lo, hi = int(np.min(lo)), int(np.max(hi))
        if hi <= lo:
            return
        self.checked += 1
        size = self.sizes[name]
        if off + lo < 0 or off + hi > size:
            self.errors.append(f"{kernel}: {name} bytes [{off + lo}, {off + hi}) outside its {size} bytes")

    def rsrc(self, kernel, ptr, base, nbytes):
        """A buffer resource at ptr + base of nbytes (arrays: one resource per element)."""
        base, nbytes = np.asarray(base, np.int64), np.asarray(nbytes, np.int64)
        if base.size == 0:
            return
        if np.any(nbytes >= 1 << 32) or np.any(nbytes < 0):
            self.errors.append(f"{kernel}: {ptr[0]} resource size {int(nbytes.max())} does not fit 32 bits")
        self.span(kernel, ptr, base.min(), (base + nbytes).max())


def at(ptr, nbytes):
    return (ptr[0], ptr[1] + int(nbytes))


# ---------------------------------------------------------------- kernels

def row_kernel(a, kernel, T, spans):
    """The one-wave-per-row kernels (embed_norm_kernel elementwise.hip:15, residual_norm_kernel :120,
    norm_split_kernel :264, the ple_*_kernel family ple.hip:30-218): row < T; loads of chunk
    min(e, width - 4) and stores of element e = c * 256 + 4 lane + j < width. spans: (pointer, bytes
    per row of the access)."""
    for ptr, row_bytes in spans:
        if ptr is not None:
            a.span(kernel, ptr, 0, T * row_bytes)


def embed_norm(a, T, D, tokens, x, h):
    row_kernel(a, "embed_norm", T, [(tokens, I32), (x, D * F32), (h, D * F16)])


def residual_norm(a, T, D, x, t16, h):
    row_kernel(a, "residual_norm", T, [(x, D * F32), (t16, D * F16), (h, D * F16)])


def norm_split(a, T, D, x, h3):
    row_kernel(a, "norm_split", T, [(x, D * F32), (h3, 3 * D * F16)])


def qk_norm_rope(a, T, H, KV, HD, qkv, positions, q, k, v, q_lo=None, k_lo=None, pos=None, table_rows=8192):
    """qk_norm_rope_kernel (elementwise.hip:327): item = (t, slot) < T (H + 2 KV); reads
    qkv[t][slot][0, HD), the RoPE row positions[t]; writes q / k / v (and the low halves)."""
    S = H + 2 * KV
    a.span("qk_norm_rope", qkv, 0, T * S * HD * F32)
    a.span("qk_norm_rope", positions, 0, T * I32)
    for p, heads in ((q, H), (k, KV), (v, KV), (q_lo, H), (k_lo, KV)):
        if p is not None:
            a.span("qk_norm_rope", p, 0, T * heads * HD * F16)
    if pos is not None and T and int(pos[:T].max()) >= table_rows:
        a.errors.append(f"qk_norm_rope: position {int(pos[:T].max())} past the {table_rows}-row RoPE table")


def vt_rows(a, kernel, vt, rows, vt_cols, vcol_used):
    """Stores vt[r][vcol[t]] for r < rows (V^T, [max_kvd][vt_cols] fp16)."""
    if vt is None or len(vcol_used) == 0:
        return
    if vcol_used.min() < 0:
        a.errors.append(f"{kernel}: negative V^T column")
    a.span(kernel, vt, 0, ((rows - 1) * vt_cols + int(vcol_used.max()) + 1) * F16)


def qkv_norm_rope_vt(a, T, H, KV, HD, qkv16, positions, q, k, v, vcol, vt_cols, vt, vc):
    """qkv_norm_rope_vt_kernel (elementwise.hip:417): token t = 64 blockIdx + 4 wave + i < T; V^T rows
    r < KV HD at column vcol[t] for t < T."""
    S = H + 2 * KV
    a.span("qkv_norm_rope_vt", qkv16, 0, T * S * HD * F16)
    a.span("qkv_norm_rope_vt", positions, 0, T * I32)
    a.span("qkv_norm_rope_vt", vcol, 0, T * I32 if vt is not None else 0)
    for p, heads in ((q, H), (k, KV), (v, KV)):
        a.span("qkv_norm_rope_vt", p, 0, T * heads * HD * F16)
    vt_rows(a, "qkv_norm_rope_vt", vt, KV * HD, vt_cols, vc[:T])


def v_transpose(a, T, width, v, vcol, vt_cols, vt, vc):
    """v_transpose_kernel (attention.hip:1294): reads v[t][c0 + cc .. + 8) for t < T, c0 + cc < width;
    writes vt[c0 + d][vcol[t]]."""
    a.span("v_transpose", v, 0, T * width * F16)
    a.span("v_transpose", vcol, 0, T * I32)
    vt_rows(a, "v_transpose", vt, width, vt_cols, vc[:T])


EPI_BYTES = {"f32": lambda N: N * F32, "f16": lambda N: N * F16, "geglu": lambda N: N // 2 * F16}


def gemm(a, kernel, M, N, K, x, y, epi):
    """launch_gemm_q8 (gemm.hip:698): gemm_kernel (:259) or gemm_skinny_kernel (:295). The activation
    resource covers X[M][K] (buffer_rsrc(X, M K 2)); stores are guarded by row < M, col < N
    (gemm_store_tile, :81), the GeGLU pairs writing column gcol / 2 of N / 2."""
    if M == 0:
        return
    a.rsrc(kernel, x, 0, M * K * F16)
    a.span(kernel, y, 0, M * EPI_BYTES[epi](N))


def gemm_qkv(a, M, N, K, hd, H, KV, x, e, pos, vc):
    """launch_gemm_qkv (gemm.hip:734): short batches take the skinny GEMM into the fp16 staging
    [M][N] and qkv_rowpass_kernel (:553), else gemm_qkv_kernel (:441); both read positions[t] and
    vcol[t] for t < M, store q / k / v rows t < M and V^T rows (slot - H - KV) HD + d at vcol[t]."""
    if M == 0:
        return
    a.rsrc("gemm_qkv", x, 0, M * K * F16)
    if e["stage"] is not None and M <= SKINNY_MAX_ROWS and K % 128 == 0:
        a.span("gemm_qkv (staging)", e["stage"], 0, M * N * F16)
    a.span("gemm_qkv", e["positions"], 0, M * I32)
    for p, heads in ((e["q"], H), (e["k"], KV), (e["v"], KV)):
        if p is not None:
            a.span("gemm_qkv", p, 0, M * heads * hd * F16)
    if e["vt"] is not None:
        a.span("gemm_qkv", e["vcol"], 0, M * I32)
        vt_rows(a, "gemm_qkv", e["vt"], KV * hd, e["vt_cols"], vc[:M])


def attention_items(a, kernel, work, H, KV, HD, q, k, vt, vt_cols, o, item_queries, q_lo=None, k_lo=None,
                    leave_empty=True):
    """attention_v2_kernel (attention.hip:291), attention_v3_kernel (:556, one workgroup per KV head or per query head) and
    attention_split_kernel (:860): per work item (seq_start, len, q0, vt_start) with len > 0 and head h, resources
        Q at (seq_start qStride + h HD) of ((len - 1) qStride + HD) halves, K likewise over kvStride,
        V^T at (kvh HD vt_cols + vt_start) of ((HD - 1) vt_cols + vt_cols - vt_start) halves,
    and output stores at row seq_start + qi for qi < min(q0 + item_queries, len). The kernels leave
    an item with len <= 0 before any access (leave_empty)."""
    w = work[work[:, 1] > 0] if leave_empty else work
    if len(w) == 0:
        return
    s, n, q0, vs = w[:, 0], w[:, 1], w[:, 2], w[:, 3]
    qS, kS = H * HD, KV * HD
    for p in (q, q_lo):
        if p is not None:
            a.rsrc(kernel, p, np.concatenate([(s * qS + h * HD) * F16 for h in (0, H - 1)]),
                   np.concatenate([((n - 1) * qS + HD) * F16] * 2))
    for p in (k, k_lo):
        if p is not None:
            a.rsrc(kernel, p, np.concatenate([(s * kS + h * HD) * F16 for h in (0, KV - 1)]),
                   np.concatenate([((n - 1) * kS + HD) * F16] * 2))
    if np.any(vs % 8):
        a.errors.append(f"{kernel}: V^T start column not a multiple of 8")
    a.rsrc(kernel, vt, np.concatenate([((kvh * HD * vt_cols) + vs) * F16 for kvh in (0, KV - 1)]),
           np.concatenate([((HD - 1) * vt_cols + vt_cols - vs) * F16] * 2))
    qend = np.minimum(q0 + item_queries, n)
    a.span(kernel, o, ((s + q0) * qS) * F16, ((s + qend) * qS) * F16)


def attention_legacy(a, work, H, KV, HD, hw, q, k, v, o, rows_alloc_k):
    """attention_kernel (attention.hip:93) with attn_stage (:52): plain loads of q rows qi < len, K and
    V key rows kb .. kb + 63 of every 64-key block from the window start (not clamped to the
    sequence: the callers keep 64 rows of slack), output rows qi < len."""
    w = work[work[:, 1] > 0]
    if len(w) == 0:
        return
    s, n, q0 = w[:, 0], w[:, 1], w[:, 2]
    qS, kS = H * HD, KV * HD
    kstart = np.zeros_like(n) if hw == 0 else np.maximum(q0 - hw, 0)
    kend = n if hw == 0 else np.minimum(q0 + ATTN_QUERIES + hw, n)
    kstart = kstart // 64 * 64
    nblocks = (kend - kstart + 63) // 64
    qend = np.minimum(q0 + 32, n)
    a.span("attention", q, (s + q0) * qS * F16, (s + qend) * qS * F16)
    a.span("attention", o, (s + q0) * qS * F16, (s + qend) * qS * F16)
    last_key = s + kstart + nblocks * 64  # one past the last key row read
    for p in (k, v):
        a.span("attention", p, (s + kstart) * kS * F16, last_key * kS * F16)


def pooled_projection(a, n_rows, width, n_out, x, out):
    """pooled_projection_kernel (elementwise.hip:630): rows r < n_rows of x [*][width] (16-byte loads
    of columns clamped to width - 4), out[r][n] for n < n_out. The weight planes are the model's."""
    a.span("pooled_projection", x, 0, n_rows * width * F32)
    a.span("pooled_projection", out, 0, n_rows * n_out * F32)


def mean_pool(a, seqs, width, x, seq_ptr, pooled):
    """mean_pool_kernel (elementwise.hip:562): rows start .. start + len - 1 of each sequence, 16-byte
    loads of columns c .. c + 3 < width."""
    a.span("mean_pool", seq_ptr, 0, len(seqs) * SEQ_BYTES)
    a.span("mean_pool", pooled, 0, len(seqs) * width * F32)
    for st, n in seqs:
        if n:
            a.span("mean_pool", x, st * width * F32, (st + n) * width * F32)


# ---------------------------------------------------------------- the forward

def stage_copies(a, b):
    """The staged arrays stage() (runtime.cpp:837) copies into the workspace."""
    n = b["n"]
    a.span("stage", ("tokens", 0), 0, n * I32)
    a.span("stage", ("positions", 0), 0, n * I32)
    a.span("stage", ("seqs", 0), 0, len(b["seqs"]) * SEQ_BYTES)
    a.span("stage", ("work", 0), 0, len(b["work"]) * WORK_BYTES)
    if len(b["work2"]):
        a.span("stage", ("work2", 0), 0, len(b["work2"]) * WORK_BYTES)
        a.span("stage", ("vcol", 0), 0, n * I32)


def replay(m, b, positions=None):
    """Replays the launches of one forward of batch b (encode, or encode_split when the plan splits
    it) and returns the Audit."""
    ws = workspace(m, b)
    a = Audit(ws)
    stage_copies(a, b)
    pos = positions if positions is not None else np.concatenate(
        [np.arange(n) for _, n in b["seqs"]] + [np.zeros(0, np.int64)]).astype(np.int64)
    if b["n_parts"] == 1:
        parts = [(0, b["n"], b["work2"], b["work"])]
    else:
        parts = [(b["part_row"][p], b["part_row"][p + 1] - b["part_row"][p],
                  b["work2"][b["part_work"][p]:b["part_work"][p + 1]], None) for p in range(b["n_parts"])]
    split = b["n_parts"] > 1
    D, H, LP = m["hidden"], m["heads"], m["layers"] * m["pl"]
    vc = b["vcol"] if b["vcol"] is not None else np.zeros(0, np.int64)
    vt_cap = b.get("vt_cap", 0)

    def rows(name, r0, width, esize):
        return (name, r0 * width * esize)

    def part_base(name, r0, width, alloc_width):
        # encode_split's part_base: the base at which absolute row r0 lands at its part's slice
        return (name, r0 * (alloc_width - width) * F16)

    for r0, T, w2, w1 in parts:
        vcp = vc[r0:r0 + T]
        embed_norm(a, T, D, rows("tokens", r0, 1, I32), rows("x", r0, D, F32), rows("h", r0, D, F16))
        if m["pl"] > 0:
            row_kernel(a, "ple_input", T, [(rows("x", r0, D, F32), D * F32), (rows("x16", r0, D, F16), D * F16),
                                           (rows("rs", r0, 1, F32), F32)])
            gemm(a, "gemm_ple_model_proj", T, LP, D, rows("x16", r0, D, F16), rows("ple", r0, LP, F32), "f32")
            row_kernel(a, "ple_norm", T * m["layers"], [(rows("ple", r0, LP, F32), m["pl"] * F32)])
            a.span("ple_norm", rows("rs", r0, 1, F32), 0, T * F32)
        for li, L in enumerate(m["layer"]):
            last = li + 1 == m["layers"]
            hd, KV, qd, kvd = L["hd"], L["kv"], L["qd"], L["kvd"]
            N = qd + 2 * kvd
            hw = m["window"] // 2 if L["sliding"] else 0
            if L["qkv_fused"]:
                e = dict(positions=rows("positions", r0, 1, I32), q=rows("q", r0, m["max_qd"], F16),
                         k=rows("k", r0, m["max_kvd"], F16),
                         v=None if (L["attn_v2"] or split) else rows("v", r0, m["max_kvd"], F16),
                         vcol=rows("vcol", r0, 1, I32), vt=("vt", 0) if L["attn_v2"] else None, vt_cols=vt_cap,
                         stage=None if split else ("qkv", 0))
                gemm_qkv(a, T, N, D, hd, H, KV, rows("h", r0, D, F16), e, pos[r0:r0 + T], vcp)
            else:
                qkv = rows("qkv", r0, m["max_qkv"], F32)
                if L["precise"]:
                    norm_split(a, T, D, rows("x", r0, D, F32), rows("h3", r0, 3 * D, F16))
                    gemm(a, "gemm_qkv", T, N, 3 * D, rows("h3", r0, 3 * D, F16), qkv, "f32")
                else:
                    gemm(a, "gemm_qkv", T, N, D, rows("h", r0, D, F16), qkv, "f16" if L["qkv_gn"] else "f32")
                q, k, v = rows("q", r0, m["max_qd"], F16), rows("k", r0, m["max_kvd"], F16), rows("v", r0, m["max_kvd"], F16)
                if L["qkv_gn"]:
                    qkv_norm_rope_vt(a, T, H, KV, hd, qkv, rows("positions", r0, 1, I32), q, k, v,
                                     rows("vcol", r0, 1, I32), vt_cap, ("vt", 0) if L["attn_v2"] else None, vcp)
                else:
                    lo = L["precise"]
                    qk_norm_rope(a, T, H, KV, hd, qkv, rows("positions", r0, 1, I32), q, k, v,
                                 rows("q_lo", r0, m["max_qd"], F16) if lo else None,
                                 rows("k_lo", r0, m["max_kvd"], F16) if lo else None, pos[r0:r0 + T], m["max_tokens"])
                    if L["attn_v2"]:
                        v_transpose(a, T, kvd, v, rows("vcol", r0, 1, I32), vt_cap, ("vt", 0), vcp)
            if L["attn_v2"]:
                if split:
                    qp, kp = part_base("q", r0, qd, m["max_qd"]), part_base("k", r0, kvd, m["max_kvd"])
                    op = part_base("attn", r0, qd, m["max_qd"])
                    qlp = part_base("q_lo", r0, qd, m["max_qd"]) if L["precise"] else None
                    klp = part_base("k_lo", r0, kvd, m["max_kvd"]) if L["precise"] else None
                else:
                    qp, kp, op = ("q", 0), ("k", 0), ("attn", 0)
                    qlp, klp = (("q_lo", 0), ("k_lo", 0)) if L["precise"] else (None, None)
                attention_items(a, "attention", w2, H, KV, hd, qp, kp, ("vt", 0), vt_cap, op, b["items"], qlp, klp)
            else:
                assert not split
                attention_legacy(a, w1, H, KV, hd, hw, ("q", 0), ("k", 0), ("v", 0), ("attn", 0), None)
            # the part's rows of t (fp32) hold two fp16 [T][D] halves: down's output in the first,
            # o's in the second (runtime.cpp encode / encode_split)
            t16 = rows("t", r0, 2 * D, F16)
            o16 = (t16[0], t16[1] + T * D * F16)
            gemm(a, "gemm_o", T, D, qd, rows("attn", r0, m["max_qd"], F16), o16, "f16")
            # residual_norm, or residual_norm_h (the same reads, h only) without the per-layer inputs
            residual_norm(a, T, D, rows("x", r0, D, F32), o16, rows("h", r0, D, F16))
            gemm(a, "gemm_gate_up", T, 2 * m["ff"], D, rows("h", r0, D, F16), rows("act", r0, m["ff"], F16), "geglu")
            gemm(a, "gemm_down", T, D, m["ff"], rows("act", r0, m["ff"], F16), t16, "f16")
            if m["pl"] > 0:
                x16, rs = rows("x16", r0, D, F16), rows("rs", r0, 1, F32)
                row_kernel(a, "ple_residual_input", T, [(rows("x", r0, D, F32), D * F32), (t16, D * F16), (x16, D * F16),
                                                        (rs, F32)])
                ple_t = rows("ple_t", r0, m["pl"], F32)
                gemm(a, "gemm_ple_gate", T, m["pl"], D, x16, ple_t, "f32")
                # ple_gate_kernel (ple.hip:171) reads ple[(row L + layer) pl .. + pl) of its part's rows
                row_kernel(a, "ple_gate", T, [(ple_t, m["pl"] * F32), (rs, F32), (rows("g16", r0, m["pl"], F16), m["pl"] * F16),
                                              (rows("rs2", r0, 1, F32), F32)])
                if T:
                    a.span("ple_gate", rows("ple", r0, LP, F32), li * m["pl"] * F32,
                           ((T - 1) * m["layers"] + li + 1) * m["pl"] * F32)
                gemm(a, "gemm_ple_proj", T, D, m["pl"], rows("g16", r0, m["pl"], F16), rows("t", r0, D, F32), "f32")
                # the last layer's norm writes fp32 rows into hn (the final norm), the others fp16 h
                hout = (rows("hn", r0, D, F32), D * F32) if last else (rows("h", r0, D, F16), D * F16)
                row_kernel(a, "ple_residual_norm", T, [(rows("x", r0, D, F32), D * F32), (rows("t", r0, D, F32), D * F32),
                                                       (rows("rs2", r0, 1, F32), F32), hout])
            else:
                row_kernel(a, "residual_norm_two", T, [(rows("x", r0, D, F32), D * F32), (o16, D * F16), (t16, D * F16),
                                                       (rows("hn", r0, D, F32), D * F32) if last else (rows("h", r0, D, F16), D * F16)])
    mean_pool(a, b["seqs"], D, ("hn", 0), ("seqs", 0), ("pooled_n", 0))
    pooled_projection(a, len(b["seqs"]), D, m["out_dims"], ("pooled_n", 0), ("pooled", 0))
    return a


def check_parts_disjoint(m, b):
    """encode_split's parts run unsynchronised: the row slices each part writes (row r0 times a
    buffer's allocated width, up to r0 + T rows) must not overlap another part's."""
    errs = []
    if b["n_parts"] < 2:
        return errs
    widths = dict(x=m["hidden"] * F32, h=m["hidden"] * F16, q=m["max_qd"] * F16, k=m["max_kvd"] * F16,
                  attn=m["max_qd"] * F16, t=m["hidden"] * F32, act=m["ff"] * F16, out=m["out_dims"] * F32,
                  qkv=m["max_qkv"] * F32, hn=m["hidden"] * F32)
    for name, wb in widths.items():
        spans = [(b["part_row"][p] * wb, b["part_row"][p + 1] * wb) for p in range(b["n_parts"])]
        for i in range(1, len(spans)):
            if spans[i][0] < spans[i - 1][1]:
                errs.append(f"parts {i - 1} and {i} overlap in {name}")
    return errs
