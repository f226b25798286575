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
