"""The vLLM V1 boundary (integration/vllm_backend.py) with stand-in vLLM
classes: routing, shape gate, install() patching, env gating. CPU only; the
GPU run of the same forward is in test_gpu_vllm.py."""

from __future__ import annotations

import types

import pytest
import torch

from integration import vllm_backend as vb
from pagedattn import flat_splits_for, plan_decode, plan_launch


class FakeBaseImpl:
    """Stands in for vLLM's TritonAttentionImpl: records delegated calls."""

    def __init__(self, num_heads=32, num_kv_heads=8, head_size=128, **extra):
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_size = head_size
        self.scale = head_size ** -0.5
        self.kv_cache_dtype = "auto"
        self.alibi_slopes = None
        self.logits_soft_cap = 0
        self.sliding_window = (-1, -1)
        self.kv_sharing_target_layer_name = None
        self.base_calls = 0
        self.__dict__.update(extra)

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None):
        self.base_calls += 1
        return "base"


class FakeBaseBackend:
    pass


def _meta(**over):
    m = types.SimpleNamespace(max_query_len=1, num_actual_tokens=2, use_cascade=False,
                              local_attn_metadata=None, max_seq_len=300,
                              block_table=torch.zeros((4, 20), dtype=torch.int32),
                              seq_lens=torch.tensor([300, 5, 0, 0], dtype=torch.int32),
                              slot_mapping=torch.tensor([299, 4], dtype=torch.int64))
    m.__dict__.update(over)
    return m


def _kv(dtype=torch.float16, nb=8):
    return torch.zeros((2, nb, 16, 8, 128), dtype=dtype)


@pytest.fixture(autouse=True)
def _reset_stats():
    for k in vb.STATS:
        vb.STATS[k] = 0
    yield


def test_supports_shape():
    assert vb.supports_shape(32, 8, 128) == (True, "")
    assert vb.supports_shape(14, 2, 64)[0]
    assert not vb.supports_shape(30, 8, 128)[0]
    assert not vb.supports_shape(32, 8, 96)[0]
    assert not vb.supports_shape(32, 0, 128)[0]


@pytest.mark.parametrize("impl_over,meta_over,kv,out,scale,expect", [
    ({}, None, "kv", "out", None, "profiling run (no metadata)"),
    ({}, {}, "kv", None, None, "no output buffer"),
    ({}, {}, "kv", "out", 1.0, "fused output quantization"),
    ({}, {}, "empty", "out", None, "empty kv cache"),
    ({"kv_cache_dtype": "fp8_e4m3"}, {}, "kv", "out", None, "fp8 kv cache"),
    ({"alibi_slopes": torch.ones(32)}, {}, "kv", "out", None, "alibi slopes"),
    ({"logits_soft_cap": 30.0}, {}, "kv", "out", None, "logits soft cap"),
    ({"sliding_window": (4095, 0)}, {}, "kv", "out", None, "sliding window"),
    ({}, {"local_attn_metadata": object()}, "kv", "out", None, "local (iRoPE) attention"),
    ({}, {"use_cascade": True}, "kv", "out", None, "cascade attention"),
    ({}, {"max_query_len": 7}, "kv", "out", None, "not a pure-decode batch"),
    ({}, {}, "f32", "out", None, "cache dtype is not fp16 or bf16"),
    ({}, {}, "kv", "out", None, ""),
])
def test_reason_to_delegate(impl_over, meta_over, kv, out, scale, expect):
    impl = FakeBaseImpl(**impl_over)
    meta = None if meta_over is None else _meta(**meta_over)
    kv_cache = {"kv": _kv(), "empty": torch.zeros(0), "f32": _kv(torch.float32)}[kv]
    output = torch.zeros(2, 32, 128, dtype=torch.float16) if out else None
    assert vb._reason_to_delegate(impl, meta, kv_cache, output, scale) == expect


def test_forward_routes(monkeypatch):
    Backend, Impl = vb.build_backend_classes(FakeBaseBackend, FakeBaseImpl)
    assert Backend.get_impl_cls() is Impl
    # the reference backend's registered name (vllm_backend.py:154-156)
    assert Backend.get_name() == vb.BACKEND_NAME == "PAGEDATTN_TRITON"
    seen = []
    monkeypatch.setattr(vb, "decode_forward", lambda *a: seen.append(a) or "ours")
    q = torch.zeros(4, 32, 128, dtype=torch.float16)
    out = torch.zeros_like(q)
    impl = Impl()
    assert impl.forward(None, q, q, q, _kv(), _meta(), out) == "ours"
    assert len(seen) == 1
    # prefill goes to vLLM
    assert impl.forward(None, q, q, q, _kv(), _meta(max_query_len=5), out) == "base"
    # unsupported head_dim goes to vLLM
    odd = Impl(head_size=96)
    assert odd.forward(None, q, q, q, _kv(), _meta(), out) == "base"
    assert vb.STATS["delegated_calls"] == 2 and impl.base_calls == 1 and odd.base_calls == 1


def test_decode_forward_builds_the_cache_view(monkeypatch):
    monkeypatch.setattr(vb, "_cu_count", lambda dev: 256)
    writes, calls = [], []

    def fake_write(layer, impl, key, value, kc, vc, slots):
        writes.append((kc.shape, vc.shape, slots.clone()))

    def fake_decode(q, cache, out, num_splits, sm_scale, max_seq_len):
        calls.append(dict(q=q, cache=cache, out=out, num_splits=num_splits, sm_scale=sm_scale,
                          max_seq_len=max_seq_len))

    impl = FakeBaseImpl()
    q = torch.randn(4, 32, 128).half()
    output = torch.zeros_like(q)
    kv = _kv()
    meta = _meta()
    res = vb.decode_forward(impl, None, q, q, q, kv, meta, output, write_kv=fake_write,
                            decode=fake_decode)
    assert res is output
    assert writes[0][0] == (8, 16, 8, 128) and torch.equal(writes[0][2], meta.slot_mapping)
    c = calls[0]
    assert c["q"].shape == (2, 32, 128) and c["out"].data_ptr() == output.data_ptr()
    cache = c["cache"]
    assert cache.k_cache.data_ptr() == kv[0].data_ptr() and cache.v_cache.data_ptr() == kv[1].data_ptr()
    assert cache.block_size == 16 and cache.kv_dtype == "fp16"
    assert cache.block_table.shape[0] == 2 and torch.equal(cache.seq_lens, meta.seq_lens[:2])
    assert (cache.shape.num_q_heads, cache.shape.num_kv_heads, cache.shape.head_dim) == (32, 8, 128)
    assert c["num_splits"] == plan_launch(2, 300, 8, 4, 256).num_splits > 1
    assert c["sm_scale"] == impl.scale and c["max_seq_len"] == 300
    assert vb.STATS == {"decode_calls": 1, "decode_tokens": 2, "delegated_calls": 0}
    # a layer sharing another layer's KV does not write
    impl.kv_sharing_target_layer_name = "model.layers.0.attn"
    vb.decode_forward(impl, None, q, q, q, kv, meta, output, write_kv=fake_write, decode=fake_decode)
    assert len(writes) == 1


def test_install_patches_once():
    class Platform:
        @classmethod
        def get_attn_backend_cls(cls, selected_backend, head_size, dtype, kv_cache_dtype,
                                 block_size, use_v1, use_mla):
            return "vllm.builtin.Backend"

    assert vb.install(Platform) == vb.QUALNAME
    assert Platform.get_attn_backend_cls(None, 128, torch.float16, "auto", 16, True, False) == vb.QUALNAME
    assert Platform.get_attn_backend_cls(None, 128, torch.float16, "auto", 16, True, True) == "vllm.builtin.Backend"
    assert Platform.get_attn_backend_cls(None, 128, torch.float16, "auto", 16, False, False) == "vllm.builtin.Backend"
    patched = Platform.__dict__["get_attn_backend_cls"]
    assert vb.install(Platform) == vb.QUALNAME
    assert Platform.__dict__["get_attn_backend_cls"] is patched


def test_maybe_install_from_env(monkeypatch):
    class Platform:
        @classmethod
        def get_attn_backend_cls(cls, *a):
            return "x"

    monkeypatch.delenv("PAGEDATTN_VLLM_BACKEND", raising=False)
    assert vb.maybe_install_from_env(Platform) is False
    assert not getattr(Platform, "_pagedattn_patched", False)
    monkeypatch.setenv("PAGEDATTN_VLLM_BACKEND", "1")
    assert vb.maybe_install_from_env(Platform) is True
    assert Platform._pagedattn_patched


def test_qualname_resolves():
    import importlib

    mod_name, cls_name = vb.QUALNAME.rsplit(".", 1)
    mod = importlib.import_module(mod_name)
    assert mod is vb and hasattr(mod, cls_name)
    assert (mod.PagedAttnTritonBackend is None) == (not vb.HAVE_VLLM)


def test_decode_forward_takes_the_flat_split_for_large_batches(monkeypatch):
    """Host-side routing only: with n * ceil(max_seq_len / 32) tiles enough
    for the flat split's waves, the step launches it (no device sync)."""
    monkeypatch.setattr(vb, "_cu_count", lambda dev: 256)
    monkeypatch.setattr(vb, "flat_waves_per_simd", lambda kv, d: 2)
    calls = []

    def fake_decode(q, cache, out, sm_scale, **kw):
        calls.append(kw)

    impl = FakeBaseImpl()
    n = 64
    q = torch.randn(n, 32, 128).half()
    meta = _meta(num_actual_tokens=n, max_seq_len=4096,
                 block_table=torch.zeros((n, 256), dtype=torch.int32),
                 seq_lens=torch.full((n,), 4096, dtype=torch.int32))
    impl.kv_sharing_target_layer_name = "shared"
    vb.decode_forward(impl, None, q, q, q, _kv(), meta, torch.zeros_like(q), decode=fake_decode)
    # a uniform batch: equal tile ranges (no per-sequence charge)
    assert calls[-1] == {"flat_splits": flat_splits_for(8, 4, 256, 2), "flat_seq_cost": 0}
    # a small step stays on the classic split
    meta = _meta(max_seq_len=300)
    vb.decode_forward(impl, None, q, q, q, _kv(), meta, torch.zeros_like(q), decode=fake_decode)
    assert calls[-1] == plan_launch(2, 300, 8, 4, 256).launch_kwargs() and "num_splits" in calls[-1]
    # so does a single long sequence (its classic merge is shorter than the flat one)
    meta = _meta(num_actual_tokens=1, max_seq_len=16384,
                 block_table=torch.zeros((1, 1024), dtype=torch.int32),
                 seq_lens=torch.full((1,), 16384, dtype=torch.int32))
    vb.decode_forward(impl, None, q[:1], q[:1], q[:1], _kv(), meta, torch.zeros_like(q[:1]),
                      decode=fake_decode)
    assert calls[-1] == {"num_splits": plan_launch(1, 16384, 8, 4, 256).num_splits, "max_seq_len": 16384}
    assert calls[-1]["num_splits"] > 1


@pytest.mark.parametrize("dtype,limit", [(torch.float16, 1024), (torch.bfloat16, 1024)],
                         ids=["fp16", "bf16"])
def test_decode_forward_runs_large_short_batches_unsplit(monkeypatch, dtype, limit):
    """Host-side routing only: a batch with 8 unsplit workgroups per CU whose
    longest sequence has at most the KV type's ragged limit runs unsplit;
    one token more takes the flat split. (The boundary serves 2-byte caches
    only, as the reference's backend does.)"""
    monkeypatch.setattr(vb, "_cu_count", lambda dev: 256)
    monkeypatch.setattr(vb, "flat_waves_per_simd", lambda kv, d: 1)
    calls = []

    def fake_decode(q, cache, out, sm_scale, **kw):
        calls.append(kw)

    impl = FakeBaseImpl()
    impl.kv_sharing_target_layer_name = "shared"
    n = 256  # 8 kv heads, group 4: 2048 workgroups = 8 per CU
    q = torch.randn(n, 32, 128).half()
    for msl, want_flat in ((limit, False), (limit + 1, True)):
        meta = _meta(num_actual_tokens=n, max_seq_len=msl,
                     block_table=torch.zeros((n, 80), dtype=torch.int32),
                     seq_lens=torch.full((n,), msl, dtype=torch.int32))
        vb.decode_forward(impl, None, q, q, q, _kv(dtype), meta, torch.zeros_like(q), decode=fake_decode)
        if want_flat:
            assert calls[-1] == {"flat_splits": flat_splits_for(8, 4, 256, 1), "flat_seq_cost": 0}
        else:
            assert calls[-1] == {"num_splits": 1, "max_seq_len": msl}
    # half the batch (4 workgroups per CU) keeps the flat split
    meta = _meta(num_actual_tokens=n // 2, max_seq_len=limit,
                 block_table=torch.zeros((n // 2, 80), dtype=torch.int32),
                 seq_lens=torch.full((n // 2,), limit, dtype=torch.int32))
    vb.decode_forward(impl, None, q[: n // 2], q[: n // 2], q[: n // 2], _kv(dtype), meta,
                      torch.zeros_like(q[: n // 2]), decode=fake_decode)
    assert calls[-1] == {"flat_splits": flat_splits_for(8, 4, 256, 1), "flat_seq_cost": 0}


def _boundary_plan(monkeypatch, lens, msl=None, host_lens=True, kv=torch.float16, shape=(32, 8, 128)):
    """The launch keywords the boundary's decode_forward picks for a step."""
    monkeypatch.setattr(vb, "_cu_count", lambda dev: 256)
    monkeypatch.setattr(vb, "flat_waves_per_simd", lambda kv_dtype, d: 1)
    calls = []

    def fake_decode(q, cache, out, sm_scale, **kw):
        calls.append(kw)

    hq, hkv, d = shape
    impl = FakeBaseImpl(num_heads=hq, num_kv_heads=hkv, head_size=d)
    impl.kv_sharing_target_layer_name = "shared"
    n = len(lens)
    t = torch.tensor(lens, dtype=torch.int32)
    extra = {"seq_lens_cpu": t} if host_lens else {}
    meta = _meta(num_actual_tokens=n, max_seq_len=msl if msl is not None else max(lens),
                 block_table=torch.zeros((n, 4), dtype=torch.int32), seq_lens=t, **extra)
    q = torch.zeros(n, hq, d, dtype=kv)
    kvc = torch.zeros((2, 4, 16, hkv, d), dtype=kv)
    vb.decode_forward(impl, None, q, q, q, kvc, meta, torch.zeros_like(q), decode=fake_decode)
    kw = dict(calls[-1])
    host = kw.pop("seq_lens_host", None)
    if host is not None:  # a flat launch planned on host lengths also takes them
        assert host_lens and kw.get("flat_splits") and host.dtype == torch.int32
        assert host.tolist() == [int(x) for x in lens]
    return kw


def _wrapper_plan(lens, kv="fp16", shape=(32, 8, 128)):
    """The launch `paged_decode_hip(num_splits=None)` plans for the same batch."""
    hq, hkv, d = shape
    return plan_launch(len(lens), 0, hkv, hq // hkv, 256, 1, kv_dtype=kv, head_dim=d,
                       seq_lens=lens).launch_kwargs()


UNIFORM = [(b, t) for b in (1, 4, 24, 32, 64, 128, 256, 512, 1024, 1100)
           for t in (16, 200, 256, 1024, 1056, 4096, 16384, 70000)]


@pytest.mark.parametrize("shape", [(32, 8, 128), (64, 8, 128), (14, 2, 64)], ids=["8b", "70b", "qwen"])
@pytest.mark.parametrize("kv", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
def test_boundary_plans_as_the_wrapper_with_host_lengths(monkeypatch, shape, kv):
    """One planner: with the step's lengths on the host (`seq_lens_cpu`), the
    boundary's launch is the one the decode wrapper plans, for uniform and
    ragged batches."""
    name = "bf16" if kv == torch.bfloat16 else "fp16"
    g = torch.Generator().manual_seed(1)
    batches = [[t] * b for b, t in UNIFORM if b * t <= 4_000_000]
    batches += [torch.randint(1, hi, (b,), generator=g).tolist()
                for b in (3, 64, 200, 512) for hi in (300, 3000, 40000) if b * hi <= 4_000_000]
    for lens in batches:
        assert _boundary_plan(monkeypatch, lens, kv=kv, shape=shape) == _wrapper_plan(lens, name, shape), \
            (len(lens), max(lens))


@pytest.mark.parametrize("shape", [(32, 8, 128), (64, 8, 128), (14, 2, 64)], ids=["8b", "70b", "qwen"])
def test_boundary_without_host_lengths_on_uniform_batches(monkeypatch, shape):
    """Metadata with device-only lengths: the boundary plans from the batch
    size and the longest length, as for a ragged batch. On uniform batches it
    then picks the wrapper's launch except where the wrapper uses what only
    the lengths tell: a nearly uniform batch that fills the CUs unsplit runs
    unsplit there (short sequences, or K/V under the per-CU byte limit),
    while the boundary keeps the flat split, which ragged batches need."""
    from pagedattn.hip_decode import _fills_unsplit

    hq, hkv, d = shape
    for b, t in UNIFORM:
        if b * t > 4_000_000:
            continue
        lens = [t] * b
        got = _boundary_plan(monkeypatch, lens, host_lens=False, shape=shape)
        want = _wrapper_plan(lens, "fp16", shape)
        if got != want:
            assert want == {"num_splits": 1, "max_seq_len": t}, (b, t, got, want)
            assert "flat_splits" in got and _fills_unsplit(lens, hkv, hq // hkv, 256), (b, t)
        # the same plan as plan_launch from (batch, max_seq_len) alone
        p = plan_launch(b, t, hkv, hq // hkv, 256, 1, kv_dtype="fp16", head_dim=d)
        assert got == p.launch_kwargs()


def test_host_seq_lens_reads_cpu_copies_only():
    assert vb._host_seq_lens(types.SimpleNamespace(), 2) is None
    assert vb._host_seq_lens(types.SimpleNamespace(seq_lens_cpu=None), 2) is None
    m = types.SimpleNamespace(seq_lens_cpu=torch.tensor([5, 6, 7], dtype=torch.int32))
    got = vb._host_seq_lens(m, 2)
    assert got.dtype == torch.int32 and got.is_contiguous() and got.tolist() == [5, 6]
    m = types.SimpleNamespace(seq_lens_cpu=torch.tensor([5, 6, 7], dtype=torch.int64))
    assert vb._host_seq_lens(m, 3).dtype == torch.int32


def test_host_seq_lens_check_catches_a_stale_copy(monkeypatch):
    """PAGEDATTN_CHECK_HOST_LENS=1 compares the host copy with seq_lens."""
    monkeypatch.setenv("PAGEDATTN_CHECK_HOST_LENS", "1")
    dev = torch.tensor([5, 6, 7], dtype=torch.int32)
    ok = types.SimpleNamespace(seq_lens=dev, seq_lens_cpu=dev.clone())
    assert vb._host_seq_lens(ok, 3).tolist() == [5, 6, 7]
    stale = types.SimpleNamespace(seq_lens=dev, seq_lens_cpu=torch.tensor([5, 6, 8], dtype=torch.int32))
    with pytest.raises(ValueError, match="stale"):
        vb._host_seq_lens(stale, 3)
    monkeypatch.delenv("PAGEDATTN_CHECK_HOST_LENS")
    assert vb._host_seq_lens(stale, 3).tolist() == [5, 6, 8]  # unchecked by default


def test_decode_step_is_planned_once_for_all_layers(monkeypatch):
    """A step's layers share its metadata: the plan is made for the first
    layer and reused by the others; a new step (new metadata) plans again.
    Planning a ragged batch of 256 on host lengths takes well under a
    millisecond (a loop per length took ~0.4 ms)."""
    import time

    monkeypatch.setattr(vb, "_cu_count", lambda dev: 256)
    monkeypatch.setattr(vb, "flat_waves_per_simd", lambda kv_dtype, d: 1)
    planned = []
    real = vb.plan_launch
    monkeypatch.setattr(vb, "plan_launch", lambda *a, **k: planned.append(1) or real(*a, **k))
    seen = []

    def fake_decode(q, cache, out, sm_scale, **kw):
        seen.append(kw)

    impl = FakeBaseImpl(num_heads=32, num_kv_heads=8, head_size=128)
    impl.kv_sharing_target_layer_name = "shared"
    g = torch.Generator().manual_seed(3)
    n = 256
    q = torch.zeros(n, 32, 128, dtype=torch.float16)
    kvc = torch.zeros((2, 4, 16, 8, 128), dtype=torch.float16)
    for step in range(3):
        t = torch.randint(1, 2048, (n,), generator=g, dtype=torch.int32)
        meta = _meta(num_actual_tokens=n, max_seq_len=int(t.max()), block_table=torch.zeros((n, 4), dtype=torch.int32),
                     seq_lens=t, seq_lens_cpu=t.clone())
        for layer in range(24):
            vb.decode_forward(impl, None, q, q, q, kvc, meta, torch.zeros_like(q), decode=fake_decode)
        assert len(planned) == step + 1
        assert all(kw == seen[-1] for kw in seen[-24:])
        assert torch.equal(seen[-1]["seq_lens_host"], t)
    lens = torch.randint(1, 2048, (n,), generator=g, dtype=torch.int32)
    t0 = time.perf_counter()
    for _ in range(20):
        real(n, 0, 8, 4, 256, 1, kv_dtype="fp16", head_dim=128, seq_lens=lens)
    assert (time.perf_counter() - t0) / 20 < 1e-3


class _NHDBackend:
    @staticmethod
    def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size):
        return (2, num_blocks, block_size, num_kv_heads, head_size)


class _FastImpl(FakeBaseImpl):
    def forward(self, layer, query, key, value, kv_cache, attn_metadata, output=None,
                output_scale=None):
        self.base_calls += 1
        return "fast-prefill"


class _PagedLayoutBackend:
    @staticmethod
    def get_kv_cache_shape(num_blocks, block_size, num_kv_heads, head_size):
        return (2, num_blocks, block_size * num_kv_heads * head_size)


@pytest.fixture
def fake_bases(monkeypatch):
    """Stand-in vLLM backend modules: rocm_aiter_fa, triton_attn and an
    `aiter` package, plus a base with the paged (non-NHD) layout."""
    aiter_mod = types.ModuleType("vllm.v1.attention.backends.rocm_aiter_fa")
    aiter_mod.AiterFlashAttentionBackend = type("AiterFlashAttentionBackend", (_NHDBackend,), {})
    aiter_mod.AiterFlashAttentionImpl = type("AiterFlashAttentionImpl", (_FastImpl,), {})
    triton_mod = types.ModuleType("vllm.v1.attention.backends.triton_attn")
    triton_mod.TritonAttentionBackend = type("TritonAttentionBackend", (_NHDBackend,), {})
    triton_mod.TritonAttentionImpl = type("TritonAttentionImpl", (FakeBaseImpl,), {})
    other = types.ModuleType("stand_in_backends")
    other.PagedBackend = _PagedLayoutBackend
    other.PagedImpl = FakeBaseImpl
    monkeypatch.setitem(__import__("sys").modules, aiter_mod.__name__, aiter_mod)
    monkeypatch.setitem(__import__("sys").modules, triton_mod.__name__, triton_mod)
    monkeypatch.setitem(__import__("sys").modules, other.__name__, other)
    # use_base rebinds module globals: restore them after the test
    for name in ("PagedAttnTritonBackend", "PagedAttnTritonImpl", "BASE_NAME"):
        monkeypatch.setattr(vb, name, getattr(vb, name))
    return aiter_mod, triton_mod


def test_prefill_backend_choice_keeps_decode_on_the_kernel(monkeypatch, fake_bases):
    aiter_mod, _ = fake_bases
    assert vb.use_base("rocm_aiter_fa") == "rocm_aiter_fa" == vb.BASE_NAME
    Backend, Impl = vb.PagedAttnTritonBackend, vb.PagedAttnTritonImpl
    assert issubclass(Backend, aiter_mod.AiterFlashAttentionBackend)
    assert issubclass(Impl, aiter_mod.AiterFlashAttentionImpl)
    assert Backend.get_name() == "PAGEDATTN_TRITON" and Backend.get_impl_cls() is Impl
    seen = []
    monkeypatch.setattr(vb, "decode_forward", lambda *a: seen.append(a) or "ours")
    q = torch.zeros(4, 32, 128, dtype=torch.float16)
    impl = Impl()
    # pure decode: the HIP kernel; prefill and mixed batches: the chosen base
    assert impl.forward(None, q, q, q, _kv(), _meta(), torch.zeros_like(q)) == "ours"
    assert impl.forward(None, q, q, q, _kv(), _meta(max_query_len=9), torch.zeros_like(q)) == "fast-prefill"
    assert len(seen) == 1 and impl.base_calls == 1
    # QUALNAME resolves to the rebuilt class
    mod_name, cls_name = vb.QUALNAME.rsplit(".", 1)
    assert getattr(__import__("importlib").import_module(mod_name), cls_name) is Backend


def test_auto_base_prefers_aiter_when_it_imports(monkeypatch, fake_bases):
    import sys

    monkeypatch.setitem(sys.modules, "aiter", types.ModuleType("aiter"))
    assert vb.resolve_base("auto")[0] == "rocm_aiter_fa"
    monkeypatch.setitem(sys.modules, "aiter", None)  # import aiter raises ImportError
    name, backend, impl = vb.resolve_base("auto")
    assert name == "triton" and backend.__name__ == "TritonAttentionBackend"
    assert vb.resolve_base(None)[0] == "triton"


def test_base_with_another_cache_layout_is_refused(fake_bases):
    with pytest.raises(ValueError, match="lays its KV cache out"):
        vb.use_base("stand_in_backends:PagedBackend:PagedImpl")
    with pytest.raises(ValueError, match="unknown base backend"):
        vb.use_base("no_such_base")
    with pytest.raises(ValueError, match="no get_kv_cache_shape"):
        vb.check_nhd_layout(FakeBaseBackend)


def test_install_with_a_prefill_backend(monkeypatch, fake_bases):
    class Platform:
        @classmethod
        def get_attn_backend_cls(cls, *a):
            return "x"

    assert vb.install(Platform, prefill_backend="rocm_aiter_fa") == vb.QUALNAME
    assert vb.BASE_NAME == "rocm_aiter_fa"
    assert Platform.get_attn_backend_cls(None, 128, torch.float16, "auto", 16, True, False) == vb.QUALNAME

    class Platform2(Platform):
        pass

    monkeypatch.setenv("PAGEDATTN_VLLM_BACKEND", "1")
    monkeypatch.setenv("PAGEDATTN_PREFILL_BACKEND", "triton")
    assert vb.maybe_install_from_env(Platform2) is True
    assert vb.BASE_NAME == "triton"
