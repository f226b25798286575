"""The C-ABI boundary without a GPU: libdsv41hip.so loads, exports every function that
include/dsv41_rocm.h declares, its descriptor layouts agree with the ctypes mirrors field by
field (offsets from gcc on the header), and invalid descriptors are rejected before any
launch with the reference's messages."""

import ctypes
import json
import re
import subprocess
from pathlib import Path

import pytest
import torch

from dsv41_rocm import _lib, sample, selected_log_probs

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dsv41_rocm.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(dsv41_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = _lib.load()
    names = declared_functions()
    assert set(names) == set(_lib.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name
    assert lib.dsv41_abi_version() == _lib.ABI_VERSION


def test_descriptor_layouts_match_header(tmp_path):
    fields = {"dsv41_sampler_desc": _lib.SamplerDesc, "dsv41_logprob_desc": _lib.LogprobDesc,
              "dsv41_logprob_grad_desc": _lib.LogprobGradDesc, "dsv41_token_tis_desc": _lib.TokenTisDesc,
              "dsv41_grpo_desc": _lib.GrpoDesc,
              "dsv41_logprob_shard_desc": _lib.LogprobShardDesc, "dsv41_logprob_combine_desc": _lib.LogprobCombineDesc,
              "dsv41_sampler_shard_desc": _lib.SamplerShardDesc, "dsv41_sampler_merge_desc": _lib.SamplerMergeDesc,
              "dsv41_sampler_full_shard_desc": _lib.SamplerFullShardDesc,
              "dsv41_sampler_full_finish_desc": _lib.SamplerFullFinishDesc}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {", 'printf("{");']
    first = True
    for cname, cls in fields.items():
        for fname, _ in cls._fields_:
            sep = "" if first else ","
            lines.append(f'printf("{sep}\\"{cname}.{fname}\\": %zu", offsetof({cname}, {fname}));')
            first = False
        lines.append(f'printf(",\\"{cname}.sizeof\\": %zu", sizeof({cname}));')
    lines += ['printf("}\\n");', "return 0; }"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    got = json.loads(subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout)
    for cname, cls in fields.items():
        for fname, _ in cls._fields_:
            assert getattr(cls, fname).offset == got[f"{cname}.{fname}"], (cname, fname)
        assert ctypes.sizeof(cls) == got[f"{cname}.sizeof"]


def _sampler_desc(**kw):
    d = _lib.SamplerDesc()
    d.struct_size = ctypes.sizeof(_lib.SamplerDesc)
    d.rows, d.vocab, d.logits_dtype, d.logits_row_stride = 4, 100, _lib.DTYPE_F32, 100
    d.logits, d.uniforms = 0x1000, 0x2000
    d.out_ids, d.out_logprob, d.out_status = 0x3000, 0x4000, 0x5000
    d.temperature, d.repetition_penalty, d.top_p = 1.0, 1.0, 1.0
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,code,msg", [
    (dict(temperature=0.0), _lib.E_INVALID, "temperature must be finite and positive"),
    (dict(temperature=float("nan")), _lib.E_INVALID, "temperature must be finite and positive"),
    (dict(top_p=0.0), _lib.E_INVALID, "top_p"),
    (dict(top_k=-1), _lib.E_INVALID, "top_k"),
    (dict(min_p=1.5), _lib.E_INVALID, "min_p"),
    (dict(repetition_penalty=0.0), _lib.E_INVALID, "repetition_penalty"),
    (dict(rows=0), _lib.E_INVALID, "shape"),
    (dict(logits_row_stride=50), _lib.E_INVALID, "stride"),
    (dict(uniforms=None), _lib.E_INVALID, "uniform"),
    (dict(vocab=(1 << 21) + 1, logits_row_stride=(1 << 21) + 1), _lib.E_UNSUPPORTED, "2^21"),
    # 2^21 masses of 2^43 (a flat row) would sum to exactly 2^64
    (dict(vocab=1 << 21, logits_row_stride=1 << 21), _lib.E_UNSUPPORTED, "2^21"),
    (dict(struct_size=8), _lib.E_ABI, "size mismatch"),
    (dict(exponentials=0x6000, exponentials_row_stride=100, top_k=5), _lib.E_UNSUPPORTED, "exponential race"),
    (dict(exponentials=0x6000, exponentials_row_stride=99), _lib.E_INVALID, "exponentials row stride"),
    (dict(replay_ids=0x7000, top_k=5), _lib.E_UNSUPPORTED, "replay_ids"),
    (dict(replay_ids=0x7000, min_p=0.1), _lib.E_UNSUPPORTED, "replay_ids"),
    (dict(replay_ids=0x7000, exponentials=0x6000, exponentials_row_stride=100), _lib.E_UNSUPPORTED, "replay_ids"),
    (dict(out_ids=None), _lib.E_INVALID, "out_ids and out_status are required"),
    (dict(out_status=None), _lib.E_INVALID, "out_ids and out_status are required"),
    # log-probs are optional, except for a replay, whose only output they are
    (dict(replay_ids=0x7000, out_logprob=None), _lib.E_INVALID, "replay_ids need out_logprob"),
])
def test_sampler_rejects_bad_descriptors_before_launch(kw, code, msg):
    lib = _lib.load()
    d = _sampler_desc(**kw)
    assert lib.dsv41_sampler_run(ctypes.byref(d), None, 0, None) == code
    assert msg in _lib.last_error()


def test_sampler_workspace_for_the_radix_path_and_deferred_selection():
    lib = _lib.load()
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(_sampler_desc())) == 0
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(_sampler_desc(top_k=5))) == 0
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(_sampler_desc(top_p=0.9))) == 4 * 100 * 4
    d = _sampler_desc(top_p=0.9)
    assert lib.dsv41_sampler_run(ctypes.byref(d), None, 0, None) == _lib.E_WORKSPACE
    # top-k batches above 256 rows hand each row's candidates (up to 256 keys and a count) to a
    # second kernel; small batches and the full-vocabulary path need nothing
    big = _sampler_desc(top_k=5, rows=300)
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(big)) == 300 * (256 * 8 + 4)
    assert lib.dsv41_sampler_run(ctypes.byref(big), None, 0, None) == _lib.E_WORKSPACE
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(_sampler_desc(top_k=5, rows=256))) == 0
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(_sampler_desc(rows=300))) == 0
    # a small top-k batch over a long vocabulary is split into 2048-aligned slices of at
    # least 6144 ids (up to about 256 workgroups, at most 4096 candidates per row): 8 rows x
    # 129280 ids -> 22 slices of 6144 ids, each (slice, row) leaving top_k keys, a count and
    # a status
    small = _sampler_desc(top_k=50, rows=8, vocab=129280, logits_row_stride=129280)
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(small)) == 22 * 8 * (50 * 8 + 4 + 4)
    assert lib.dsv41_sampler_run(ctypes.byref(small), None, 0, None) == _lib.E_WORKSPACE
    # top_k 256 caps the slices at 4096 // 256 = 16
    wide = _sampler_desc(top_k=256, rows=8, vocab=129280, logits_row_stride=129280)
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(wide)) == 16 * 8 * (256 * 8 + 4 + 4)
    # above top_k 256 the rows stay whole
    assert lib.dsv41_sampler_workspace_bytes(ctypes.byref(_sampler_desc(top_k=257, rows=8, vocab=129280,
                                                                        logits_row_stride=129280))) == 0


def _logprob_desc(**kw):
    d = _lib.LogprobDesc()
    d.struct_size = ctypes.sizeof(_lib.LogprobDesc)
    d.n_tokens, d.hidden, d.vocab = 10, 64, 300
    d.x, d.x_row_stride, d.w, d.w_row_stride = 0x1000, 64, 0x2000, 64
    d.targets, d.out_logprob, d.temperature = 0x3000, 0x4000, 1.0
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,code,msg", [
    (dict(temperature=-1.0), _lib.E_INVALID, "temperature must be finite and positive"),
    (dict(hidden=60, x_row_stride=64, w_row_stride=64), _lib.E_UNSUPPORTED, "multiple of 8"),
    (dict(x_row_stride=60), _lib.E_INVALID, "stride"),
    (dict(x=0x1008), _lib.E_INVALID, "aligned"),
    (dict(out_ratio=0x5000), _lib.E_INVALID, "behavior"),
    (dict(behavior=0x6000, is_cap=0.0), _lib.E_INVALID, "is_cap"),
])
def test_logprob_rejects_bad_descriptors_before_launch(kw, code, msg):
    lib = _lib.load()
    d = _logprob_desc(**kw)
    assert lib.dsv41_logprob_run(ctypes.byref(d), None, 0, None) == code
    assert msg in _lib.last_error()


def test_logprob_workspace_and_empty_batch():
    lib = _lib.load()
    d = _logprob_desc()
    ws = lib.dsv41_logprob_workspace_bytes(ctypes.byref(d))
    assert ws > 0 and ws % (16 * 10) == 0  # splits x tokens x 16-byte states
    assert lib.dsv41_logprob_run(ctypes.byref(d), None, 0, None) == _lib.E_WORKSPACE
    empty = _logprob_desc(n_tokens=0)
    assert lib.dsv41_logprob_run(ctypes.byref(empty), None, 0, None) == _lib.OK


def _grad_desc(**kw):
    d = _lib.LogprobGradDesc()
    d.struct_size = ctypes.sizeof(_lib.LogprobGradDesc)
    d.n_tokens, d.hidden, d.vocab = 10, 64, 300
    d.x, d.x_row_stride, d.w, d.w_row_stride = 0x1000, 64, 0x2000, 64
    d.targets, d.lse, d.temperature = 0x3000, 0x4000, 1.0
    d.vocab_begin, d.vocab_end, d.out, d.out_row_stride = 0, 300, 0x5000, 304
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,code,msg", [
    (dict(temperature=0.0), _lib.E_INVALID, "temperature must be finite and positive"),
    (dict(vocab_begin=10, vocab_end=10), _lib.E_INVALID, "vocabulary range"),
    (dict(vocab_end=301), _lib.E_INVALID, "vocabulary range"),
    (dict(out_row_stride=296), _lib.E_INVALID, "output row stride"),
    (dict(out_row_stride=302), _lib.E_INVALID, "output row stride"),
    (dict(out=0x5008), _lib.E_INVALID, "aligned"),
    (dict(grad_entropy=0x6000), _lib.E_INVALID, "entropies"),
    (dict(lse=None), _lib.E_INVALID, "lse"),
    (dict(hidden=60, x_row_stride=64, w_row_stride=64), _lib.E_UNSUPPORTED, "multiple of 8"),
    (dict(struct_size=16), _lib.E_ABI, "size mismatch"),
])
def test_logprob_grad_rejects_bad_descriptors_before_launch(kw, code, msg):
    lib = _lib.load()
    d = _grad_desc(**kw)
    assert lib.dsv41_logprob_grad_run(ctypes.byref(d), None) == code
    assert msg in _lib.last_error()
    empty = _grad_desc(n_tokens=0)
    assert lib.dsv41_logprob_grad_run(ctypes.byref(empty), None) == _lib.OK


def test_python_entry_points_fail_loudly_off_gpu():
    with pytest.raises(ValueError, match="GPU"):
        sample(torch.zeros(2, 10))
    with pytest.raises(ValueError, match="temperature"):
        sample(torch.zeros(2, 10), temperature=0.0)
    with pytest.raises(ValueError, match="GPU"):
        selected_log_probs(torch.zeros(3, 8, dtype=torch.bfloat16), torch.zeros(5, 8, dtype=torch.bfloat16),
                           torch.zeros(3, dtype=torch.int64))
    from dsv41_rocm import full_shard_draw, full_shard_finish, full_shard_masses, full_shard_states
    with pytest.raises(ValueError, match="GPU"):
        full_shard_states(torch.zeros(2, 10), vocab_offset=0, vocab_size=10)
    with pytest.raises(ValueError, match="GPU"):
        full_shard_masses(torch.zeros(2, 10), torch.zeros(1, 2, 4, dtype=torch.int64), shard_index=0,
                          vocab_offset=0, vocab_size=10)
    with pytest.raises(ValueError, match="GPU"):
        full_shard_draw(torch.zeros(2, 10), torch.zeros(1, 2, 4, dtype=torch.int64), shard_index=0,
                        vocab_offset=0, vocab_size=10, uniforms=torch.zeros(2))
    with pytest.raises(ValueError, match="draw must be"):
        full_shard_finish(torch.zeros(1, 2, 4, dtype=torch.int64), vocab_size=10, draw="top_p")
    with pytest.raises(ValueError, match=r"\[n_shards, rows, 4\]"):
        full_shard_finish(torch.zeros(2, 4, dtype=torch.int64), vocab_size=10, draw="greedy")


def test_custom_ops_registered_with_fake_kernels():
    from torch._subclasses.fake_tensor import FakeTensorMode

    import dsv41_rocm  # noqa: F401

    assert hasattr(torch.ops.dsv41_rocm, "sample_rows")
    assert hasattr(torch.ops.dsv41_rocm, "selected_log_probs")
    with FakeTensorMode():
        x = torch.empty(4, 100, device="meta")
        ids, lps, kept, st = torch.ops.dsv41_rocm.sample_rows(x, torch.empty(4, device="meta"), None, None,
                                                              0.7, 1.0, 0.0, 0.0, 0, 1.0, 0.0, False)
        assert ids.shape == (4,) and ids.dtype == torch.int64 and lps.dtype == torch.float32
        assert kept.dtype == st.dtype == torch.int32
        h = torch.empty(5, 16, dtype=torch.bfloat16, device="meta")
        w = torch.empty(30, 16, dtype=torch.bfloat16, device="meta")
        t = torch.empty(5, dtype=torch.int64, device="meta")
        lp, ent, ratio, lse = torch.ops.dsv41_rocm.selected_log_probs(h, w, t, 1.0, None, 2.0)
        assert lp.shape == ent.shape == lse.shape == (5,) and ratio.shape == (0,)
        lp, ent, ratio, _ = torch.ops.dsv41_rocm.selected_log_probs(h, w, t, 1.0, torch.empty(5, device="meta"), 2.0)
        assert ratio.shape == (5,)


def test_custom_ops_have_no_cpu_kernel():
    import dsv41_rocm  # noqa: F401

    with pytest.raises(NotImplementedError):
        torch.ops.dsv41_rocm.sample_rows(torch.zeros(2, 10), torch.rand(2), None, None,
                                         1.0, 1.0, 0.0, 0.0, 0, 1.0, 0.0, False)


def _shard_desc(sampler, **kw):
    d = _lib.SamplerShardDesc()
    d.struct_size = ctypes.sizeof(_lib.SamplerShardDesc)
    d.max_candidates = 5
    d.sampler = ctypes.pointer(sampler)
    d.vocab_offset, d.vocab_size = 100, 400
    d.out_keys, d.out_counts, d.out_status = 0x7000, 0x8000, 0x9000
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("skw,kw,code,msg", [
    (dict(top_k=0), {}, _lib.E_UNSUPPORTED, "needs 1 <= top_k <= 2048"),
    (dict(top_k=3000), dict(max_candidates=3000), _lib.E_UNSUPPORTED, "needs 1 <= top_k <= 2048"),
    (dict(top_k=5, top_p=0.9, min_p=0.0), dict(max_candidates=4), _lib.E_INVALID, "max_candidates"),
    (dict(top_k=5), dict(vocab_offset=350), _lib.E_INVALID, "within a vocabulary"),
    (dict(top_k=5), dict(out_keys=None), _lib.E_INVALID, "out_keys"),
    (dict(top_k=5, exponentials=0x6000, exponentials_row_stride=100), {}, _lib.E_UNSUPPORTED, "exponential"),
    (dict(top_k=5), dict(struct_size=8), _lib.E_ABI, "size mismatch"),
])
def test_sampler_shard_rejects_bad_descriptors(skw, kw, code, msg):
    lib = _lib.load()
    base = _sampler_desc(uniforms=None, out_ids=None, out_logprob=None, **skw)  # a slice needs neither
    d = _shard_desc(base, **kw)
    assert lib.dsv41_sampler_shard_run(ctypes.byref(d), None) == code
    assert msg in _lib.last_error()


def _merge_desc(**kw):
    d = _lib.SamplerMergeDesc()
    d.struct_size = ctypes.sizeof(_lib.SamplerMergeDesc)
    d.rows, d.n_shards, d.max_candidates = 4, 8, 64
    d.keys, d.counts, d.status, d.uniforms = 0x1000, 0x2000, 0x3000, 0x4000
    d.top_k, d.top_p, d.min_p = 64, 1.0, 0.0
    d.out_ids, d.out_logprob, d.out_status = 0x5000, 0x6000, 0x7000
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("kw,code,msg", [
    (dict(rows=0), _lib.E_INVALID, "must be positive"),
    (dict(top_k=0), _lib.E_INVALID, "top_k must be in [1, 2048]"),
    (dict(top_p=1.5), _lib.E_INVALID, "top_p"),
    (dict(uniforms=None), _lib.E_INVALID, "uniform"),
    (dict(keys=None), _lib.E_INVALID, "keys, counts"),
    (dict(n_shards=64, max_candidates=2048, top_k=2048), _lib.E_UNSUPPORTED, "candidate buffer"),
    (dict(struct_size=8), _lib.E_ABI, "size mismatch"),
])
def test_sampler_merge_rejects_bad_descriptors(kw, code, msg):
    lib = _lib.load()
    d = _merge_desc(**kw)
    assert lib.dsv41_sampler_merge_run(ctypes.byref(d), None) == code
    assert msg in _lib.last_error()


def _full_shard_desc(sampler, **kw):
    d = _lib.SamplerFullShardDesc()
    d.struct_size = ctypes.sizeof(_lib.SamplerFullShardDesc)
    d.sampler = ctypes.pointer(sampler)
    d.vocab_offset, d.vocab_size = 100, 400
    d.n_shards, d.shard_index = 3, 1
    d.states, d.out_states, d.out_picks = 0x7000, 0x8000, 0x9000
    d.masses, d.out_masses = 0xA000, 0xB000
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("step,skw,kw,code,msg", [
    ("state", dict(top_p=0.9), {}, _lib.E_UNSUPPORTED, "no top-k, top-p or min-p"),
    ("state", dict(top_k=5), {}, _lib.E_UNSUPPORTED, "no top-k, top-p or min-p"),
    ("state", dict(min_p=0.1), {}, _lib.E_UNSUPPORTED, "no top-k, top-p or min-p"),
    ("state", {}, dict(vocab_offset=350), _lib.E_INVALID, "within a vocabulary"),
    ("state", {}, dict(out_states=None), _lib.E_INVALID, "out_states"),
    ("state", {}, dict(struct_size=8), _lib.E_ABI, "size mismatch"),
    ("state", dict(replay_ids=0x6000), {}, _lib.E_UNSUPPORTED, "replay_ids"),
    ("draw", {}, dict(shard_index=3), _lib.E_INVALID, "shard_index"),
    ("draw", {}, dict(states=None), _lib.E_INVALID, "gathered states"),
    ("draw", {}, dict(out_picks=None), _lib.E_INVALID, "out_picks"),
    ("draw", {}, dict(masses=None), _lib.E_INVALID, "gathered masses"),
    ("draw", dict(uniforms=None), {}, _lib.E_INVALID, "one uniform per row"),
    ("draw", dict(greedy=1), {}, _lib.E_INVALID, "greedy rows need no draw step"),
    ("mass", {}, dict(out_masses=None), _lib.E_INVALID, "out_masses"),
    ("mass", {}, dict(states=None), _lib.E_INVALID, "gathered states"),
    ("mass", {}, dict(shard_index=-1), _lib.E_INVALID, "shard_index"),
    ("mass", dict(greedy=1), {}, _lib.E_INVALID, "greedy rows need no draw step"),
    ("mass", dict(top_k=3), {}, _lib.E_UNSUPPORTED, "no top-k, top-p or min-p"),
])
def test_sampler_full_shard_rejects_bad_descriptors(step, skw, kw, code, msg):
    lib = _lib.load()
    base = _sampler_desc(out_ids=None, out_logprob=None, out_status=None, **skw)
    d = _full_shard_desc(base, **kw)
    run = {"state": lib.dsv41_sampler_full_state_run, "mass": lib.dsv41_sampler_full_mass_run,
           "draw": lib.dsv41_sampler_full_draw_run}[step]
    assert run(ctypes.byref(d), None) == code
    assert msg in _lib.last_error()


@pytest.mark.parametrize("kw,code,msg", [
    (dict(draw=3), _lib.E_INVALID, "draw must be"),
    (dict(picks=None), _lib.E_INVALID, "picks"),
    (dict(uniforms=None), _lib.E_INVALID, "one uniform per row"),
    (dict(rows=0), _lib.E_INVALID, "must be positive"),
    (dict(out_ids=None), _lib.E_INVALID, "out_ids"),
    (dict(struct_size=8), _lib.E_ABI, "size mismatch"),
])
def test_sampler_full_finish_rejects_bad_descriptors(kw, code, msg):
    lib = _lib.load()
    d = _lib.SamplerFullFinishDesc()
    d.struct_size = ctypes.sizeof(_lib.SamplerFullFinishDesc)
    d.rows, d.n_shards, d.draw = 4, 2, _lib.FULL_DRAW_CDF
    d.states, d.picks, d.uniforms, d.vocab_size = 0x1000, 0x2000, 0x3000, 400
    d.out_ids, d.out_logprob, d.out_status = 0x4000, 0x5000, 0x6000
    for k, v in kw.items():
        setattr(d, k, v)
    assert lib.dsv41_sampler_full_finish_run(ctypes.byref(d), None) == code
    assert msg in _lib.last_error()


def _integration_stub():
    """The first python block of INTEGRATION.md's ctypes section, the binding a maintainer copies."""
    text = (ROOT / "INTEGRATION.md").read_text()
    section = text.split("## 1. The ctypes binding", 1)[1]
    return section.split("```python\n", 1)[1].split("```", 1)[0]


def test_integration_stub_matches_the_binding(monkeypatch):
    # The stub loads the library by a path relative to the repository root, checks the ABI
    # version and the sampler descriptor's size, and binds every entry point it names.
    monkeypatch.chdir(ROOT)
    ns = {}
    exec(compile(_integration_stub(), "INTEGRATION.md", "exec"), ns)
    pairs = {"SamplerDesc": _lib.SamplerDesc, "LogprobDesc": _lib.LogprobDesc,
             "LogprobGradDesc": _lib.LogprobGradDesc, "GrpoDesc": _lib.GrpoDesc,
             "TokenTisDesc": _lib.TokenTisDesc}
    for name, cls in pairs.items():
        stub = ns[name]
        assert [f for f, _ in stub._fields_] == [f for f, _ in cls._fields_], name
        assert ctypes.sizeof(stub) == ctypes.sizeof(cls), name
        for fname, _ in cls._fields_:
            assert getattr(stub, fname).offset == getattr(cls, fname).offset, (name, fname)
    assert ns["lib"].dsv41_abi_version() == _lib.ABI_VERSION
    bound = set(re.findall(r"\blib\.(dsv41_[a-z_]+)\.", _integration_stub()))
    assert bound <= set(_lib.EXPORTS)
    assert "dsv41_sampler_run_static" in bound
