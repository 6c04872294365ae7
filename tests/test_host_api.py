"""CPU checks of the host-side mirror: metadata building, backend descriptor, hot-set choice, argument validation,
and the oracle's fast_topk.local / merge restatement (brute force on tiny rows, and local + merge == top-k)."""
import itertools

import numpy as np
import pytest
import torch

from oracle import spmla_ref as ref


def test_backend_descriptor():
    from arcagi2_flashnext_dots3_amd import dsa
    B = dsa.PortableSparseBackend
    assert B.get_name() == "DOTS3_PORTABLE_MLA_SPARSE"
    assert B.get_impl_cls() is dsa.PortableSparseImpl
    assert B.get_builder_cls() is dsa.PortableXPUBuilder
    assert B.get_metadata_cls() is dsa.SparseMetadata
    assert B.get_supported_head_sizes() == []


def test_builder_req_id_per_token():
    from arcagi2_flashnext_dots3_amd.dsa import CommonAttentionMetadata, PortableXPUBuilder
    qsl = torch.tensor([0, 3, 3, 7, 8], dtype=torch.int32)           # request 1 has no tokens
    cam = CommonAttentionMetadata(query_start_loc=qsl, num_reqs=4, num_actual_tokens=8, max_query_len=4,
                                  max_seq_len=100, slot_mapping=torch.arange(8),
                                  block_table_tensor=torch.zeros(4, 2, dtype=torch.int32))
    b = PortableXPUBuilder(64, 2048, 12, "cpu")
    md = b.build(0, cam)
    assert md.req_id_per_token.tolist() == [0, 0, 0, 2, 2, 2, 2, 3]
    assert b.req_id_per_token_buffer[8:].tolist() == [3, 3, 3, 3]     # padding tokens clamp to the last request
    assert md.num_decode_tokens == 8 and md.block_size == 64 and md.topk_tokens == 2048


def test_impl_rejects_unsupported_shapes():
    from arcagi2_flashnext_dots3_amd.dsa import PortableSparseImpl
    with pytest.raises(ValueError):
        PortableSparseImpl(128, 512, 0.1, 1, None, None, "fp8_ds_mla", None, "decoder", None)
    with pytest.raises(NotImplementedError):
        PortableSparseImpl(128, 576, 0.1, 1, None, 128, "fp8_ds_mla", None, "decoder", None)


def test_hot_rows_by_frequency():
    from arcagi2_flashnext_dots3_amd.sparse_offload import hot_rows_by_frequency
    counts = torch.tensor([3, 0, 5, 3, 1, 5, 0, 3])
    assert hot_rows_by_frequency(counts, 4).tolist() == [2, 5, 0, 3]   # ties -> lower row id
    assert hot_rows_by_frequency(counts, 100).tolist() == [2, 5, 0, 3, 7, 4]


def test_shard_store_validates_layout():
    from arcagi2_flashnext_dots3_amd.shard_indexer import ShardStore
    st = ShardStore(torch.zeros(10, 64, 132, dtype=torch.uint8), 1, 0)
    assert (st.BS, st.RPB, st.STRIDE_BLK, st.R_local) == (64, 64, 64 * 132, 640)
    st4 = ShardStore(torch.zeros(10, 64, 33, dtype=torch.uint8), 4, 1)     # [blocks, BS, 132 / P]
    assert (st4.RPB, st4.R_local) == (16, 160)
    with pytest.raises(ValueError):
        ShardStore(torch.zeros(10, 64, 128, dtype=torch.uint8), 1, 0)


def _brute_local(x, ctx, rank, P, kl):
    rows, Lc = x.shape
    pk = np.zeros((rows, 2 * kl), dtype=np.float32)
    pos = pk[:, kl:].view(np.int32)
    for r in range(rows):
        n = min(Lc, -(-(int(ctx[r]) - rank) // P)) if ctx[r] > rank else 0
        key = [int(ref.okey(np.float32(v))) for v in x[r, :n]]
        order = sorted(range(n), key=lambda j: (-key[j], j))[:kl]
        chosen = sorted(order)
        for s, j in enumerate(chosen):
            pk[r, s] = x[r, j]
            pos[r, s] = j * P + rank
        for s in range(len(chosen), kl):
            pk[r, s] = -np.inf
            pos[r, s] = s * P + rank
    return pk


def test_oracle_topk_local_brute_force():
    g = np.random.RandomState(3)
    for trial, (rank, P) in enumerate([(0, 1), (1, 2), (3, 4), (0, 3)]):
        x = np.round(g.randn(5, 23).astype(np.float32) * 2) / 2          # ties
        x[0, 3] = np.nan
        x[1, 4] = np.inf
        x[2, 5] = -0.0
        x[2, 6] = 0.0
        ctx = np.array([80, 23 * P, 7, 0, rank + 1], dtype=np.int32)
        for kl in (1, 6, 23, 30):
            a = ref.topk_local(x, ctx, rank, P, kl)
            b = _brute_local(x, ctx, rank, P, kl)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (trial, kl)


def test_oracle_topk_merge_brute_force_and_composition():
    g = np.random.RandomState(4)
    n, P, kl = 3, 3, 5
    allp = np.zeros((P * n, 2 * kl), dtype=np.float32)
    allp[:, :kl] = np.round(g.randn(P * n, kl) * 2) / 2
    allp[0, 1] = -np.inf
    allp[4, 2] = np.inf
    allp[:, kl:] = g.randint(0, 1000, (P * n, kl)).astype(np.int32).view(np.float32)
    for kk, tt in itertools.product((1, 7, 15), (15, 18)):
        got = ref.topk_merge(allp, n, P, kl, kk, tt)
        for r in range(n):
            cand = [(allp[p * n + r, i], p * kl + i, allp[p * n + r, kl + i:kl + i + 1].view(np.int32)[0])
                    for p in range(P) for i in range(kl)]
            cand.sort(key=lambda c: (-int(ref.okey(np.float32(c[0]))), c[1]))
            exp = [(-1 if np.isinf(v) else int(pos)) for v, _, pos in cand[:kk]] + [-1] * (tt - kk)
            assert got[r].tolist() == exp
    # local + merge at P = 1 is the exact top-k
    x = np.round(g.randn(4, 200).astype(np.float32) * 3) / 3
    ctx = np.array([200, 150, 20, 0], dtype=np.int32)
    pk = ref.topk_local(x, ctx, 0, 1, 64)
    assert np.array_equal(ref.topk_merge(pk, 4, 1, 64, 64, 64), ref.topk(x, ctx, 64))


def test_host_pool_capacity_guard(monkeypatch):
    """A pinned host pool beyond ARC_OFFLOAD_HOST_FRAC (default half) of the available host memory is refused before
    anything is pinned; within it, nothing is raised."""
    from arcagi2_flashnext_dots3_amd import sparse_offload as so
    avail = so.host_memory_available()                    # this host's MemAvailable
    assert avail is None or avail > 0
    monkeypatch.delenv("ARC_OFFLOAD_HOST_FRAC", raising=False)
    so.check_host_budget(4 << 30, available=10 << 30)
    with pytest.raises(RuntimeError, match="exceeds 50%"):
        so.check_host_budget(6 << 30, available=10 << 30)
    monkeypatch.setenv("ARC_OFFLOAD_HOST_FRAC", "0.8")
    so.check_host_budget(6 << 30, available=10 << 30)
    monkeypatch.setattr(so, "host_memory_available", lambda: 1 << 20)   # the constructor checks before pinning
    with pytest.raises(RuntimeError, match="host pool"):
        so.LayerOffload(1 << 20, "cpu")


def test_packed_option_rejects_caches_it_cannot_stage():
    """packed=True (request-packed MTP decode) stages union rows from the static hot set's Row656 lines or the host
    pool; the W-way cache and compact cache lines are refused before anything is allocated."""
    from arcagi2_flashnext_dots3_amd import sparse_offload as so
    with pytest.raises(ValueError, match="packed"):
        so.LayerOffload(1024, "cpu", cache_rows=64, cache_mode="ways", ways=16, packed=True)
    with pytest.raises(ValueError, match="packed"):
        so.LayerOffload(1024, "cpu", cache_rows=64, row_fmt="e2m2", cache_fmt="e2m2", packed=True)


def test_verify_outputs_reports_bad_tokens():
    """ARC_OFFLOAD_VERIFY's comparison: per token max |a - b| / max(max |b|, 1e-3); a planted error on one token is
    reported, agreeing tokens are not, and the statistics accumulate over calls."""
    from arcagi2_flashnext_dots3_amd.diagnostics import verify_outputs
    g = torch.Generator().manual_seed(0)
    ref_o = torch.randn(5, 4, 16, generator=g)
    test_o = ref_o + 1e-4 * torch.randn(5, 4, 16, generator=g)
    test_o[2, 1, 3] += 0.5 * ref_o[2].abs().max()                       # token 2 off by half its largest value
    lines, st = [], {}
    rel = verify_outputs(test_o, ref_o, st, label="L3", log=lines.append)
    assert (rel > 0.1).nonzero().flatten().tolist() == [2]
    assert st["calls"] == 1 and st["tokens"] == 5 and st["bad"] == 1 and 0.49 < st["max_rel"] < 0.51
    assert len(lines) == 1 and "bad=1" in lines[0] and "first=[2]" in lines[0]
    verify_outputs(ref_o, ref_o, st, log=lines.append)
    assert st["calls"] == 2 and st["bad"] == 1 and len(lines) == 1


def test_topk_check_recall():
    """ARC_SHARD_CHECK's statistic: recall of a selection against torch.topk over the row's first ctx columns."""
    from arcagi2_flashnext_dots3_amd.diagnostics import TopkCheck
    lg = torch.arange(20, dtype=torch.float32).flip(0).repeat(2, 1)      # column j holds 19 - j
    lg[1, 3] = float("-inf")
    ctx = torch.tensor([20, 10])
    lines = []
    chk = TopkCheck(every=2, log=lines.append)
    got = torch.tensor([[0, 1, 2, 3], [0, 1, 2, 5]], dtype=torch.int32)
    r = chk.check(lg, ctx, got, 4)
    # row 0: exact; row 1: reference {0, 1, 2, 4} (column 3 is -inf), got {0, 1, 2, 5}: 3 of 4
    assert abs(r - (1.0 + 0.75) / 2) < 1e-9 and chk.min_recall == 0.75
    assert lines and "mean recall=0.87500" in lines[0]


def test_access_trace_window_and_file_layout(tmp_path):
    """ARC_OFFLOAD_DUMP's record: nothing before after_s or below min_T tokens; then store slots (kind 0) and attend
    rows (kind 1) until `calls` attend calls, saved as kinds / C / W / R / T / e<i> in an npz; unique mode keeps the
    sorted distinct valid rows and the step's slots passed to attend."""
    from arcagi2_flashnext_dots3_amd.diagnostics import AccessTrace
    now = [100.0]
    lines = []
    tr = AccessTrace(tmp_path / "whole", calls=2, after_s=5.0, min_t=2, clock=lambda: now[0], log=lines.append)
    idx = torch.tensor([[3, -1, 3], [7, 1, 2]], dtype=torch.int64)
    tr.access(idx, 2, 8, 1, 16)                                     # before after_s: nothing
    now[0] = 106.0
    tr.access(idx[:1], 1, 8, 1, 16)                                 # T below min_T: nothing
    tr.stored(torch.tensor([9]))                                    # not recording yet: nothing
    tr.access(idx, 2, 8, 1, 16)
    tr.stored(torch.tensor([4, 5]))
    tr.access(idx + 1, 2, 8, 1, 16)
    assert tr.done and len(lines) == 2 and "T=2 C=8 W=1 R=16" in lines[0]
    z = np.load(tmp_path / "whole.npz")
    assert z["kinds"].tolist() == [1, 0, 1] and int(z["C"]) == 8 and int(z["W"]) == 1 and int(z["R"]) == 16
    assert int(z["T"]) == 2 and z["e0"].dtype == np.int32
    assert np.array_equal(z["e0"], idx.numpy()) and z["e1"].tolist() == [4, 5] and np.array_equal(z["e2"], idx.numpy() + 1)
    tr.access(idx, 2, 8, 1, 16)                                     # after the window: ignored
    assert len(lines) == 2

    tu = AccessTrace(tmp_path / "uniq", calls=1, unique=True, log=lines.append)
    tu.access(idx, 2, 8, 4, 16, slots=torch.tensor([11, 12]))
    z = np.load(tmp_path / "uniq.npz")
    assert z["kinds"].tolist() == [0, 1] and z["e0"].tolist() == [11, 12] and z["e1"].tolist() == [1, 2, 3, 7]
    assert int(z["W"]) == 4
    with pytest.raises(ValueError):
        AccessTrace(tmp_path / "x", calls=0)


def test_access_trace_switches():
    """ARC_OFFLOAD_DUMP=path,after_s,calls,min_T with ARC_OFFLOAD_DUMP_LAYERS picking backbone layers by their key
    (path_L<n>, unique rows) or, without it, the first layer built; only device index 0 records."""
    from arcagi2_flashnext_dots3_amd.diagnostics import AccessTrace
    env = {"ARC_OFFLOAD_DUMP": "/tmp/d,2.5,7,3"}
    assert AccessTrace.from_env(env={}) is None
    t = AccessTrace.from_env(key="model.layers.4.attn.indexer", device="cuda:0", env=env)
    assert t.path == "/tmp/d" and t.left == 7 and t.min_t == 3 and not t.unique
    assert AccessTrace.from_env(device="cuda:0", first=False, env=env) is None
    assert AccessTrace.from_env(device="cuda:1", env=env) is None
    env["ARC_OFFLOAD_DUMP_LAYERS"] = "1,17"
    assert AccessTrace.from_env(key="model.layers.4.attn", env=env) is None
    t = AccessTrace.from_env(key="model.layers.17.attn", first=False, env=env)
    assert t.path == "/tmp/d_L17" and t.unique


def test_auto_split_respects_the_split_kernel_row_limit():
    """auto_split never picks a split whose rows per split pass the split kernel's limit (2048 rows, whole tiles of
    32): the unsplit head-group kernel takes any K."""
    from arcagi2_flashnext_dots3_amd import kernels
    assert kernels.ATTN_SPLIT_ROWS == 2048
    for T in (1, 2, 7, 23):
        for K in (64, 256, 2048, 4096, 16384, 16385, 20000, 65536):
            s = kernels.auto_split(T, 128, K)
            assert 1 <= s <= 8
            if s > 1:
                assert -(-(-(-K // s)) // 32) * 32 <= kernels.ATTN_SPLIT_ROWS
    assert kernels.auto_split(1, 128, 16384) == 8 and kernels.auto_split(1, 128, 16385) == 1
    assert kernels.auto_split(1, 128, 20000) == 1
    # below fused_max_tokens tokens auto_split may take the split merge (needs a workspace), never at or above it
    for H in (16, 64, 128):
        Tm = kernels.fused_max_tokens(H)
        assert kernels.auto_split(Tm, H, 4096) > 1 and kernels.auto_split(Tm + 1, H, 4096) == 1


def test_workspace_under_capture_reuses_the_eager_one(monkeypatch):
    """Under HIP graph capture the workspace cache allocates nothing: it hands out the device's largest eager
    workspace of the kind and raises when there is none or it is too small (a buffer allocated inside a capture holds
    its contents only after the first replay). Grown buffers stay referenced, so captured graphs keep valid ones."""
    from arcagi2_flashnext_dots3_amd import kernels
    monkeypatch.setattr(kernels, "_WS", {})
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    d0, d1 = torch.device("cuda:0"), torch.device("cuda:1")
    with pytest.raises(ValueError, match="graph capture"):
        kernels._workspace("attn", d0, 1000)
    small, big, other = torch.empty(512, dtype=torch.uint8), torch.empty(4096, dtype=torch.uint8), \
        torch.empty(1 << 20, dtype=torch.uint8)
    kernels._WS[("attn", d0, 1)] = small
    kernels._WS[("attn", d0, 2)] = big
    kernels._WS[("attn", d1, 1)] = other          # another device's buffer is never used
    kernels._WS[("topk", d0, 1)] = other          # nor another kind's
    b, key = kernels._workspace("attn", d0, 1000)
    assert b is big and key is None
    with pytest.raises(ValueError, match="graph capture"):
        kernels._workspace("attn", d0, 5000)
