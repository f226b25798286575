"""dsv41_sampler_run_static (the sampler entry point that allocates nothing, with its
workspace in a static device array) against dsv41_sampler_run with a caller workspace, through
the C ABI.  Same kernels, so every output must be identical bit for bit.  Two calls in a row
share the array; the second is smaller, so stale contents of the first would show."""

import ctypes

import pytest
import torch

from dsv41_rocm import _lib, workloads
from dsv41_rocm.sampling import _rows_desc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _desc(inp, outs):
    logits, history, uniforms, knobs = inp["logits"], inp["history"], inp["uniforms"], inp["knobs"]
    d = _rows_desc(logits, history, None, knobs.get("temperature", 1.0), knobs.get("repetition_penalty", 1.0),
                   knobs.get("presence_penalty", 0.0), knobs.get("frequency_penalty", 0.0), knobs.get("top_k", 0),
                   knobs.get("top_p", 1.0), knobs.get("min_p", 0.0))
    d.uniforms = uniforms.data_ptr()
    d.greedy = 0
    d.out_ids, d.out_logprob, d.out_kept, d.out_status = (t.data_ptr() for t in outs)
    return d


def _outs(rows):
    return (torch.full((rows,), -7, dtype=torch.int64, device=DEV), torch.full((rows,), 7.0, device=DEV),
            torch.full((rows,), -7, dtype=torch.int32, device=DEV), torch.full((rows,), -7, dtype=torch.int32,
                                                                                device=DEV))


def _run_both(inp):
    lib = _lib.load()
    rows = inp["logits"].shape[0]
    stream = torch.cuda.current_stream(DEV).cuda_stream
    ref, got = _outs(rows), _outs(rows)
    dr, dg = _desc(inp, ref), _desc(inp, got)
    ws_bytes = lib.dsv41_sampler_workspace_bytes(ctypes.byref(dr))
    assert 0 < ws_bytes <= _lib.SAMPLER_STATIC_SCRATCH_BYTES
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    _lib.check(lib.dsv41_sampler_run(ctypes.byref(dr), ws.data_ptr(), ws_bytes, stream))
    _lib.check(lib.dsv41_sampler_run_static(ctypes.byref(dg), stream))
    torch.cuda.synchronize()
    for a, b in zip(ref, got):
        assert torch.equal(a, b)
    assert int(got[3].max()) == 0 and int(got[0].min()) >= 0
    return ws_bytes


@pytest.mark.parametrize("first,second", [(("E", 512), ("E", 300)), (("E", 400), ("A", 8)),
                                          (("E", 2200), ("E", 2100))])
def test_static_scratch_matches_workspace_entry_point(first, second):
    sizes = []
    for name, rows in (first, second):
        print(f"case: dsv41_sampler_run_static config {name} rows={rows}", flush=True)
        sizes.append(_run_both(workloads.sampler_inputs(name, rows=rows, device=DEV)))
    assert sizes[1] < sizes[0]


def test_static_scratch_rejects_batches_above_its_size():
    # top-p alone takes the radix path, whose workspace is rows * vocab * 4 bytes
    rows, vocab = 64, 151936
    assert rows * vocab * 4 > _lib.SAMPLER_STATIC_SCRATCH_BYTES
    logits = torch.zeros(rows, vocab, device=DEV)
    inp = dict(logits=logits, history=None, uniforms=torch.zeros(rows, device=DEV), knobs=dict(top_p=0.9))
    outs = _outs(rows)
    rc = _lib.load().dsv41_sampler_run_static(ctypes.byref(_desc(inp, outs)),
                                             torch.cuda.current_stream(DEV).cuda_stream)
    assert rc == _lib.E_UNSUPPORTED and "static maximum" in _lib.last_error()


def _flat_rows_inputs(rows, knobs, seed):
    """fp32 rows of config E's vocabulary; every third row flat, so that a min-p bound keeps
    the whole row (more survivors than the internal bound: those rows take the fallback)."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(rows, 151936, generator=g)
    logits[::3] = 0.0
    return dict(logits=logits.to(DEV), history=None, uniforms=torch.rand(rows, generator=g).to(DEV), knobs=knobs)


def test_static_scratch_top_p_alone_then_min_p_fallback_rows():
    # top-p alone on 32 rows keeps one fp32 z row per row in the scratch (19.4 MB); min-p
    # alone then runs the internal top-k bound, and its flat rows go to generic_kernel,
    # whose z rows follow in the same array
    sizes = []
    for rows, knobs, seed in ((32, dict(top_p=0.9, temperature=0.8), 1), (12, dict(min_p=0.05), 2)):
        print(f"case: dsv41_sampler_run_static rows={rows} knobs={knobs}", flush=True)
        sizes.append(_run_both(_flat_rows_inputs(rows, knobs, seed)))
    assert sizes[1] < sizes[0]


def test_static_scratch_replays_under_graph_capture():
    # The entry point allocates and clears nothing, so a captured launch replays as is.
    lib = _lib.load()
    inp = workloads.sampler_inputs("E", rows=300, device=DEV)
    rows = 300
    ref, got = _outs(rows), _outs(rows)
    stream = torch.cuda.current_stream(DEV).cuda_stream
    _lib.check(lib.dsv41_sampler_run_static(ctypes.byref(_desc(inp, ref)), stream))
    torch.cuda.synchronize()
    dg = _desc(inp, got)
    side = torch.cuda.Stream(DEV)
    side.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(side):  # warm-up off the default stream, as capture requires
        _lib.check(lib.dsv41_sampler_run_static(ctypes.byref(dg), side.cuda_stream))
    torch.cuda.current_stream(DEV).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    print("case: dsv41_sampler_run_static under graph capture, E 300 rows", flush=True)
    with torch.cuda.graph(graph):
        rc = lib.dsv41_sampler_run_static(ctypes.byref(dg), torch.cuda.current_stream(DEV).cuda_stream)
    _lib.check(rc)
    for _ in range(3):
        for t in got:
            t.fill_(-5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(ref, got):
            assert torch.equal(a, b)
