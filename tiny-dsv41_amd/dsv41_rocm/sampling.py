"""Token sampling on MI355X: the drop-in for the sampling step of ``generate_group``.

Reference (paths relative to the Tiny-DSV41 tree):

* ``dsv41_train/rl/rollout.py:144-150`` — ``log_probs = log_softmax(logits.float() / T)``,
  non-finite check (:145-146, ``ValueError("generation log probabilities contain non-finite
  values")``), ``multinomial`` draw with a CPU generator (:148), ``behavior = log_probs[token]``.
* ``dsv41_train/rl/algorithm.py:19-21`` — ``validate_temperature``.
* ``rollout_manager/backends/vllm_actor.py:178-185, :260`` — the SamplingParams knobs
  (repetition / presence / frequency penalty, top-k, top-p, min-p) and processed log-probs.

The draw is an inverse CDF in vocabulary order against one uniform per row.  Uniforms come
from the caller or from a CPU ``torch.Generator`` (``torch.rand``), so a generator state
persisted like the reference's (``rollout_manager/backends/pytorch_rl.py:70-72, :113-114``)
replays the same tokens.  All arithmetic runs in libdsv41hip.so; this module validates
arguments, allocates outputs with torch and launches on the current HIP stream.
"""

from __future__ import annotations

import math
import threading
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib


@dataclass
class SampleResult:
    """Per-row outputs: drawn ids (int64), their log-probs under the processed
    distribution (fp32; None when not requested), kept-set sizes (int32) and status bits
    (int32)."""

    ids: torch.Tensor
    logprobs: Optional[torch.Tensor]
    kept: torch.Tensor
    status: torch.Tensor


def validate_temperature(temperature: float) -> None:
    """Same rule and message as algorithm.py:19-21."""
    if not math.isfinite(temperature) or temperature <= 0:
        raise ValueError("temperature must be finite and positive")


def _device_ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _status_error(status: torch.Tensor) -> None:
    bits = 0
    for v in status.cpu().tolist():
        bits |= int(v)
    if bits & _lib.STATUS_NONFINITE:
        raise ValueError("generation log probabilities contain non-finite values")
    if bits & _lib.STATUS_BAD_HISTORY:
        raise ValueError("history token ID is outside the model vocabulary")
    if bits & _lib.STATUS_BAD_UNIFORM:
        raise ValueError("uniforms must lie in [0, 1)")
    if bits & _lib.STATUS_BAD_TARGET:
        raise ValueError("target token ID is outside the model vocabulary")
    if bits & _lib.STATUS_BAD_SLICES:
        raise ValueError("gathered slice masses do not match the draw step's inputs")


def _rows_in(logits, history, history_lens, temperature, top_k):
    """Validated, GPU-resident logits [rows, V] and history of one batch."""
    validate_temperature(temperature)
    if not isinstance(logits, torch.Tensor) or logits.ndim != 2 or 0 in logits.shape:
        raise ValueError("logits must have shape [rows, vocabulary_size]")
    if not logits.is_cuda:
        raise ValueError("logits must be on the GPU (libdsv41hip has no CPU path)")
    if logits.dtype not in (torch.float32, torch.bfloat16):
        logits = logits.float()
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    if isinstance(top_k, bool) or not isinstance(top_k, int) or top_k < 0:
        raise ValueError("top_k must be a nonnegative integer")
    rows = logits.shape[0]
    if history is not None:
        if history.ndim != 2 or history.shape[0] != rows:
            raise ValueError("history must have shape [rows, history_length]")
        history = history.to(device=logits.device, dtype=torch.int64)
        if history.stride(1) != 1:
            history = history.contiguous()
        if history_lens is not None:
            history_lens = history_lens.to(device=logits.device, dtype=torch.int32).contiguous()
            if history_lens.shape != (rows,):
                raise ValueError("history_lens must have one length per row")
    return logits, history, history_lens


def _prompt_lens(history_prompt_lens, history, rows, device):
    """Per-row count of leading history entries that belong to the prompt (int32 on the
    device), or None."""
    if history_prompt_lens is None:
        return None
    if history is None:
        raise ValueError("history_prompt_lens requires a history")
    t = torch.as_tensor(history_prompt_lens).to(device=device, dtype=torch.int32).reshape(-1).contiguous()
    if t.shape != (rows,):
        raise ValueError("history_prompt_lens must have one length per row")
    return t


def _rows_desc(logits, history, history_lens, temperature, repetition_penalty, presence_penalty,
               frequency_penalty, top_k, top_p, min_p) -> _lib.SamplerDesc:
    desc = _lib.SamplerDesc()
    desc.struct_size = _lib.ctypes.sizeof(_lib.SamplerDesc)
    desc.rows, desc.vocab = logits.shape
    desc.logits_dtype = _lib.DTYPE_F32 if logits.dtype == torch.float32 else _lib.DTYPE_BF16
    desc.logits_row_stride = logits.stride(0)
    desc.logits = logits.data_ptr()
    if history is not None and history.shape[1] > 0:
        desc.history = history.data_ptr()
        desc.history_row_stride = history.stride(0)
        desc.hist_len = history.shape[1]
        desc.history_lens = _device_ptr(history_lens)
    desc.temperature = temperature
    desc.repetition_penalty = repetition_penalty
    desc.presence_penalty = presence_penalty
    desc.frequency_penalty = frequency_penalty
    desc.top_k = top_k
    desc.top_p = top_p
    desc.min_p = min_p
    return desc


def sample(
    logits: torch.Tensor,
    *,
    temperature: float = 1.0,
    uniforms: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
    history: Optional[torch.Tensor] = None,
    history_lens: Optional[torch.Tensor] = None,
    history_prompt_lens: Optional[torch.Tensor] = None,
    repetition_penalty: float = 1.0,
    presence_penalty: float = 0.0,
    frequency_penalty: float = 0.0,
    top_k: int = 0,
    top_p: float = 1.0,
    min_p: float = 0.0,
    greedy: bool = False,
    check: bool = True,
    exponentials: Optional[torch.Tensor] = None,
    logprobs: bool = True,
) -> SampleResult:
    """Sample one token per row of ``logits[rows, vocab]`` (fp32 or bf16, on the GPU).

    ``history[rows, L]`` (int64, negative = padding) feeds the penalties; ``history_lens``
    (int32 [rows]) optionally gives ragged lengths.  With ``history_prompt_lens`` (int32
    [rows]) the first entries of each row are the prompt's ids and the penalties follow vLLM:
    repetition for ids of the prompt or the output, frequency and presence for the generated
    ids only (counted among the entries past the prompt).  ``uniforms`` (fp32 [rows] in [0, 1))
    drive the draw; when omitted they are drawn with ``torch.rand(rows, generator=generator)``
    on the CPU.  With ``check`` the call synchronises and raises the reference's
    ``ValueError`` for non-finite rows, bad uniforms, or a history id at or above the
    vocabulary size; history is read only when a penalty is active (repetition != 1,
    presence or frequency != 0), so with neutral penalties such an id is ignored and not
    flagged.

    ``exponentials`` (fp32 ``[rows, vocab]`` of Exp(1) variates) switches the draw to the
    exponential race ``argmax(p / E)``, which is what ``torch.multinomial(p, 1)`` computes on
    the CPU; fed the variates of ``torch.empty(V).exponential_(1, generator=g)`` it returns
    the reference's token (rollout.py:147-148) and leaves ``g`` where the reference leaves it.
    Only without top-k / top-p / min-p.

    ``logprobs=False`` leaves the log-probs out (``SampleResult.logprobs`` is None); a greedy
    draw without truncation then forms no masses at all, only each row's first maximum
    (the reference's greedy, ``sft_eval.py:64``, is an argmax).
    """
    logits, history, history_lens = _rows_in(logits, history, history_lens, temperature, top_k)
    rows, vocab = logits.shape
    device = logits.device
    if exponentials is not None and not greedy:
        exponentials = exponentials.to(device=device, dtype=torch.float32)
        if exponentials.ndim != 2 or exponentials.shape != logits.shape:
            raise ValueError("exponentials must have the shape of logits")
        if exponentials.stride(1) != 1:
            exponentials = exponentials.contiguous()
        uniforms = torch.zeros(rows, dtype=torch.float32, device=device) if uniforms is None else uniforms
    if not greedy:
        if uniforms is None:
            if generator is not None and generator.device.type != "cpu":
                raise ValueError("generation requires a CPU torch.Generator")
            uniforms = torch.rand(rows, generator=generator, dtype=torch.float32)
        uniforms = uniforms.to(device=device, dtype=torch.float32).contiguous()
        if uniforms.shape != (rows,):
            raise ValueError("one uniform is required per row")
    ids = torch.empty(rows, dtype=torch.int64, device=device)
    lps = torch.empty(rows, dtype=torch.float32, device=device) if logprobs else None
    kept = torch.empty(rows, dtype=torch.int32, device=device)
    status = torch.empty(rows, dtype=torch.int32, device=device)
    desc = _rows_desc(logits, history, history_lens, temperature, repetition_penalty, presence_penalty,
                      frequency_penalty, top_k, top_p, min_p)
    plens = _prompt_lens(history_prompt_lens, history, logits.shape[0], logits.device)
    desc.history_prompt_lens = _device_ptr(plens)
    desc.uniforms = _device_ptr(uniforms)
    desc.greedy = 1 if greedy else 0
    desc.out_ids = ids.data_ptr()
    desc.out_logprob = _device_ptr(lps)
    desc.out_kept = kept.data_ptr()
    desc.out_status = status.data_ptr()
    if exponentials is not None and not greedy:
        desc.exponentials = exponentials.data_ptr()
        desc.exponentials_row_stride = exponentials.stride(0)
    lib = _lib.load()
    ws_bytes = lib.dsv41_sampler_workspace_bytes(_lib.ctypes.byref(desc))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_sampler_run(_lib.ctypes.byref(desc), _device_ptr(workspace), ws_bytes, stream)
    _lib.check(rc)
    if check:
        if bool((status != 0).any()):
            _status_error(status)
    return SampleResult(ids, lps, kept, status)


def sample_next(logits: torch.Tensor, temperature: float,
                generator: Optional[torch.Generator] = None, draw: str = "inverse_cdf",
                **knobs) -> tuple[int, float]:
    """Drop-in for rollout.py:144-150 on one ``[V]`` (or ``[1, V]``) logits row.

    Returns ``(token, behavior_log_prob)`` like the reference's ``token`` /
    ``float(log_probs[token])``.  ``draw="inverse_cdf"`` takes one uniform from
    ``torch.rand(1, generator=generator)``; ``draw="exponential_race"`` takes the V variates of
    ``torch.empty(V).exponential_(1, generator=generator)``, exactly what the reference's
    ``torch.multinomial(probabilities, 1, generator=generator)`` consumes, and so draws the
    reference's token and leaves the generator in the reference's state.
    """
    row = logits.reshape(1, -1) if logits.ndim == 1 else logits
    if row.ndim != 2 or row.shape[0] != 1:
        raise ValueError("model next_token_logits must return [1, vocabulary_size]")
    if draw == "inverse_cdf" and not knobs and isinstance(row, torch.Tensor) and row.is_cuda and \
            row.dtype in (torch.float32, torch.bfloat16) and row.stride(1) == 1 and row.shape[1] > 0:
        return _next_step(row, temperature, generator)
    if draw == "exponential_race":
        if generator is not None and generator.device.type != "cpu":
            raise ValueError("generation requires a CPU torch.Generator")
        e = torch.empty(1, row.shape[1], dtype=torch.float32).exponential_(1, generator=generator)
        result = sample(row, temperature=temperature, exponentials=e, **knobs)
    elif draw == "inverse_cdf":
        result = sample(row, temperature=temperature, generator=generator, **knobs)
    else:
        raise ValueError("draw must be 'inverse_cdf' or 'exponential_race'")
    return int(result.ids.item()), float(result.logprobs.item())


class _StepBuffers:
    """The batch-1 sampling step's buffers for one (device, dtype, vocabulary): a 32-byte
    pinned host block the kernel reads its uniform from and writes its outputs to (id int64,
    log-prob fp32, kept int32, status int32, uniform fp32), the device workspace and the
    descriptor.  One synchronisation per token, no copies and no allocations."""

    def __init__(self, row: torch.Tensor):
        self.host = torch.zeros(8, dtype=torch.int32, pin_memory=True)
        self.i64 = self.host.numpy().view("int64")
        self.i32 = self.host.numpy()
        self.f32 = self.host.numpy().view("float32")
        base = self.host.data_ptr()
        desc = _rows_desc(row, None, None, 1.0, 1.0, 0.0, 0.0, 0, 1.0, 0.0)
        desc.uniforms = base + 20
        desc.out_ids, desc.out_logprob, desc.out_kept, desc.out_status = base, base + 8, base + 12, base + 16
        self.desc = desc
        self.lib = _lib.load()
        self.ws_bytes = self.lib.dsv41_sampler_workspace_bytes(_lib.ctypes.byref(desc))
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=row.device)
        self.lock = threading.Lock()  # callers on several threads take turns on the block


_step_buffers: dict = {}


def _next_step(row: torch.Tensor, temperature: float, generator: Optional[torch.Generator]) -> tuple[int, float]:
    """sample_next's inverse-CDF step on one GPU row without further knobs: the kernels of
    :func:`sample` (so the same token and log-prob bit for bit) with the uniform taken from
    the generator as ``sample`` takes it."""
    validate_temperature(temperature)
    if generator is not None and generator.device.type != "cpu":
        raise ValueError("generation requires a CPU torch.Generator")
    key = (row.device, row.dtype, row.shape[1], row.stride(0), row.data_ptr() % 16 == 0)
    buf = _step_buffers.get(key)
    if buf is None:
        buf = _step_buffers[key] = _StepBuffers(row)
    u = float(torch.rand(1, generator=generator, dtype=torch.float32)[0])
    with buf.lock, torch.cuda.device(row.device):
        buf.f32[5] = u
        buf.i32[4] = -1
        d = buf.desc
        d.logits = row.data_ptr()
        d.temperature = temperature
        stream = torch.cuda.current_stream(row.device)
        rc = buf.lib.dsv41_sampler_run(_lib.ctypes.byref(d), buf.ws.data_ptr(), buf.ws_bytes, stream.cuda_stream)
        _lib.check(rc)
        stream.synchronize()
        status, token, lp = int(buf.i32[4]), int(buf.i64[0]), float(buf.f32[2])
    if status:
        _status_error(torch.tensor([status]))
    return token, lp


@dataclass
class ShardCandidates:
    """What one vocabulary slice contributes to a sharded batch, and what one all-gather
    carries: the slice's candidate keys (int64 [rows, capacity], the bit patterns of the u64
    keys of ``dsv41_sampler_shard_desc``), their counts (int32 [rows]) and the status bits
    the slice saw (int32 [rows])."""

    keys: torch.Tensor
    counts: torch.Tensor
    status: torch.Tensor


def sample_shard(
    logits: torch.Tensor,
    *,
    vocab_offset: int,
    vocab_size: int,
    top_k: int,
    temperature: float = 1.0,
    history: Optional[torch.Tensor] = None,
    history_lens: Optional[torch.Tensor] = None,
    history_prompt_lens: Optional[torch.Tensor] = None,
    repetition_penalty: float = 1.0,
    presence_penalty: float = 0.0,
    frequency_penalty: float = 0.0,
    top_p: float = 1.0,
    min_p: float = 0.0,
) -> ShardCandidates:
    """First half of sampling a vocabulary-sharded batch: this GPU's logits cover the ids
    ``[vocab_offset, vocab_offset + logits.shape[1])`` of a ``vocab_size`` vocabulary (a
    tensor-parallel head), the knobs are the batch's, and ``history`` holds global ids.
    Returns the slice's exact local top-k under its local min-p bound; gather the results of
    all slices and finish with :func:`merge_shards`.  Needs 1 <= top_k <= 2048 (the lists
    then bound what the exchange carries)."""
    logits, history, history_lens = _rows_in(logits, history, history_lens, temperature, top_k)
    rows, width = logits.shape
    if top_k < 1:
        raise ValueError("vocabulary-sharded sampling needs top_k >= 1")
    if not (0 <= vocab_offset and vocab_offset + width <= vocab_size):
        raise ValueError("the slice must lie within the vocabulary")
    device = logits.device
    keys = torch.empty(rows, top_k, dtype=torch.int64, device=device)
    counts = torch.empty(rows, dtype=torch.int32, device=device)
    status = torch.empty(rows, dtype=torch.int32, device=device)
    desc = _rows_desc(logits, history, history_lens, temperature, repetition_penalty, presence_penalty,
                      frequency_penalty, top_k, top_p, min_p)
    plens = _prompt_lens(history_prompt_lens, history, logits.shape[0], logits.device)
    desc.history_prompt_lens = _device_ptr(plens)
    shard = _lib.SamplerShardDesc()
    shard.struct_size = _lib.ctypes.sizeof(_lib.SamplerShardDesc)
    shard.max_candidates = top_k
    shard.sampler = _lib.ctypes.pointer(desc)
    shard.vocab_offset = vocab_offset
    shard.vocab_size = vocab_size
    shard.out_keys, shard.out_counts, shard.out_status = keys.data_ptr(), counts.data_ptr(), status.data_ptr()
    lib = _lib.load()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_sampler_shard_run(_lib.ctypes.byref(shard), stream)
    _lib.check(rc)
    return ShardCandidates(keys, counts, status)


def merge_shards(
    shards: list[ShardCandidates],
    *,
    top_k: int,
    top_p: float = 1.0,
    min_p: float = 0.0,
    uniforms: Optional[torch.Tensor] = None,
    generator: Optional[torch.Generator] = None,
    greedy: bool = False,
    check: bool = True,
) -> SampleResult:
    """Second half of sampling a vocabulary-sharded batch: the exact final selection (min-p,
    top-k, top-p, draw) over the gathered candidate lists, with the knobs of the
    :func:`sample_shard` calls.  Returns what :func:`sample` returns for the unsharded
    logits; uniforms and checks behave as there."""
    if not shards:
        raise ValueError("merge_shards needs the lists of at least one slice")
    keys = torch.stack([s.keys for s in shards]).contiguous()
    counts = torch.stack([s.counts for s in shards]).contiguous()
    status = torch.stack([s.status for s in shards]).contiguous()
    n_shards, rows, cap = keys.shape
    device = keys.device
    if not greedy:
        if uniforms is None:
            if generator is not None and generator.device.type != "cpu":
                raise ValueError("generation requires a CPU torch.Generator")
            uniforms = torch.rand(rows, generator=generator, dtype=torch.float32)
        uniforms = uniforms.to(device=device, dtype=torch.float32).contiguous()
        if uniforms.shape != (rows,):
            raise ValueError("one uniform is required per row")
    ids = torch.empty(rows, dtype=torch.int64, device=device)
    lps = torch.empty(rows, dtype=torch.float32, device=device)
    kept = torch.empty(rows, dtype=torch.int32, device=device)
    out_status = torch.empty(rows, dtype=torch.int32, device=device)
    d = _lib.SamplerMergeDesc()
    d.struct_size = _lib.ctypes.sizeof(_lib.SamplerMergeDesc)
    d.rows, d.n_shards, d.max_candidates = rows, n_shards, cap
    d.keys, d.counts, d.status = keys.data_ptr(), counts.data_ptr(), status.data_ptr()
    d.uniforms = _device_ptr(uniforms if not greedy else None)
    d.top_k, d.top_p, d.min_p, d.greedy = top_k, top_p, min_p, 1 if greedy else 0
    d.out_ids, d.out_logprob, d.out_kept, d.out_status = (ids.data_ptr(), lps.data_ptr(), kept.data_ptr(),
                                                          out_status.data_ptr())
    lib = _lib.load()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_sampler_merge_run(_lib.ctypes.byref(d), stream)
    _lib.check(rc)
    if check:
        if bool((out_status != 0).any()):
            _status_error(out_status)
    return SampleResult(ids, lps, kept, out_status)


def full_shard_states(
    logits: torch.Tensor,
    *,
    vocab_offset: int,
    vocab_size: int,
    temperature: float = 1.0,
    history: Optional[torch.Tensor] = None,
    history_lens: Optional[torch.Tensor] = None,
    history_prompt_lens: Optional[torch.Tensor] = None,
    repetition_penalty: float = 1.0,
    presence_penalty: float = 0.0,
    frequency_penalty: float = 0.0,
) -> torch.Tensor:
    """Step 1 of a full-vocabulary draw (no top-k, top-p or min-p: the reference's training
    mode, ``rollout.py:144-148``) over a vocabulary-sharded batch.  This GPU's logits cover the
    ids ``[vocab_offset, vocab_offset + logits.shape[1])`` of a ``vocab_size`` vocabulary and
    ``history`` holds global ids.  Returns the slice's state per row, int64 ``[rows, 4]`` (the
    32-byte ``dsv41_full_state``: its largest processed logit, status bits, its mass in a fixed
    order and its first argmax).  Gather the states of all slices (slices in vocabulary order)
    for :func:`full_shard_draw` and :func:`full_shard_finish`."""
    logits, history, history_lens = _rows_in(logits, history, history_lens, temperature, 0)
    rows, width = logits.shape
    if not (0 <= vocab_offset and vocab_offset + width <= vocab_size):
        raise ValueError("the slice must lie within the vocabulary")
    device = logits.device
    states = torch.empty(rows, _lib.FULL_STATE_BYTES // 8, dtype=torch.int64, device=device)
    desc = _rows_desc(logits, history, history_lens, temperature, repetition_penalty, presence_penalty,
                      frequency_penalty, 0, 1.0, 0.0)
    plens = _prompt_lens(history_prompt_lens, history, logits.shape[0], logits.device)
    desc.history_prompt_lens = _device_ptr(plens)
    d = _lib.SamplerFullShardDesc()
    d.struct_size = _lib.ctypes.sizeof(_lib.SamplerFullShardDesc)
    d.sampler = _lib.ctypes.pointer(desc)
    d.vocab_offset, d.vocab_size = vocab_offset, vocab_size
    d.out_states = states.data_ptr()
    lib = _lib.load()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_sampler_full_state_run(_lib.ctypes.byref(d), stream)
    _lib.check(rc)
    return states


def _gathered(parts, words: int, what: str) -> torch.Tensor:
    t = torch.stack(list(parts)) if isinstance(parts, (list, tuple)) else parts
    if t.ndim != 3 or t.shape[2] != words or t.dtype != torch.int64:
        raise ValueError(f"{what} must be the int64 [n_shards, rows, {words}] gathered from every slice")
    return t.contiguous()


def _shard_desc(logits, history, history_lens, temperature, repetition_penalty, presence_penalty,
                frequency_penalty, vocab_offset, vocab_size, states, shard_index, history_prompt_lens=None):
    """Descriptor of one slice for the mass and draw steps, with the gathered states."""
    rows, width = logits.shape
    if not (0 <= vocab_offset and vocab_offset + width <= vocab_size):
        raise ValueError("the slice must lie within the vocabulary")
    st = _gathered(states, _lib.FULL_STATE_BYTES // 8, "states").to(logits.device)
    if st.shape[1] != rows:
        raise ValueError("states must hold one state per row of every slice")
    if not 0 <= shard_index < st.shape[0]:
        raise ValueError("shard_index must name one of the gathered slices")
    desc = _rows_desc(logits, history, history_lens, temperature, repetition_penalty, presence_penalty,
                      frequency_penalty, 0, 1.0, 0.0)
    plens = _prompt_lens(history_prompt_lens, history, logits.shape[0], logits.device)
    desc.history_prompt_lens = _device_ptr(plens)
    d = _lib.SamplerFullShardDesc()
    d.struct_size = _lib.ctypes.sizeof(_lib.SamplerFullShardDesc)
    d.n_shards = st.shape[0]
    d.vocab_offset, d.vocab_size = vocab_offset, vocab_size
    d.shard_index = shard_index
    d.states = st.data_ptr()
    return d, desc, st, plens


def full_shard_masses(
    logits: torch.Tensor,
    states,
    *,
    shard_index: int,
    vocab_offset: int,
    vocab_size: int,
    temperature: float = 1.0,
    history: Optional[torch.Tensor] = None,
    history_lens: Optional[torch.Tensor] = None,
    history_prompt_lens: Optional[torch.Tensor] = None,
    repetition_penalty: float = 1.0,
    presence_penalty: float = 0.0,
    frequency_penalty: float = 0.0,
) -> torch.Tensor:
    """Step 2 of a full-vocabulary inverse-CDF draw over slices: with every slice's state
    gathered (``states``: a list in slice order, or int64 ``[n_shards, rows, 4]``), this slice's
    exact fixed-point mass ``sum_i floor(2^43 exp(z_i - M))`` against the row's maximum ``M``
    over all slices.  Returns int64 ``[rows]`` (the bits of the u64 masses); gather them from
    every slice for :func:`full_shard_draw`.  The exponential race skips this step."""
    logits, history, history_lens = _rows_in(logits, history, history_lens, temperature, 0)
    d, desc, st, plens = _shard_desc(logits, history, history_lens, temperature, repetition_penalty,
                                     presence_penalty, frequency_penalty, vocab_offset, vocab_size, states,
                                     shard_index, history_prompt_lens)
    masses = torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
    d.sampler = _lib.ctypes.pointer(desc)
    d.out_masses = masses.data_ptr()
    lib = _lib.load()
    with torch.cuda.device(logits.device):
        stream = torch.cuda.current_stream(logits.device).cuda_stream
        rc = lib.dsv41_sampler_full_mass_run(_lib.ctypes.byref(d), stream)
    _lib.check(rc)
    return masses


def full_shard_draw(
    logits: torch.Tensor,
    states,
    masses=None,
    *,
    shard_index: int,
    vocab_offset: int,
    vocab_size: int,
    temperature: float = 1.0,
    uniforms: Optional[torch.Tensor] = None,
    exponentials: Optional[torch.Tensor] = None,
    history: Optional[torch.Tensor] = None,
    history_lens: Optional[torch.Tensor] = None,
    history_prompt_lens: Optional[torch.Tensor] = None,
    repetition_penalty: float = 1.0,
    presence_penalty: float = 0.0,
    frequency_penalty: float = 0.0,
) -> torch.Tensor:
    """Step 3 of a full-vocabulary draw over slices, with every slice's state gathered
    (``states``: a list in slice order, or int64 ``[n_shards, rows, 4]``).  Inverse CDF (against
    ``uniforms``, the same fp32 ``[rows]`` on every slice): with every slice's exact mass
    gathered too (``masses``: a list of the int64 ``[rows]`` of :func:`full_shard_masses`, or
    ``[n_shards, rows]``), the slice whose masses hold the target places the token, exactly as
    the unsharded sampler would.  Exponential race (``exponentials``: this slice's columns of
    the rows' Exp(1) variates, which reproduce ``torch.multinomial``): each slice reports its
    best ``p / E`` over its columns.  Returns int64 ``[rows, 2]`` (the 16-byte
    ``dsv41_full_pick``) for :func:`full_shard_finish`.  Greedy rows need no draw step."""
    logits, history, history_lens = _rows_in(logits, history, history_lens, temperature, 0)
    rows = logits.shape[0]
    device = logits.device
    d, desc, st, plens = _shard_desc(logits, history, history_lens, temperature, repetition_penalty,
                                     presence_penalty, frequency_penalty, vocab_offset, vocab_size, states,
                                     shard_index, history_prompt_lens)
    ms = None
    if exponentials is not None:
        exponentials = exponentials.to(device=device, dtype=torch.float32)
        if exponentials.shape != logits.shape:
            raise ValueError("exponentials must have the shape of this slice's logits")
        if exponentials.stride(1) != 1:
            exponentials = exponentials.contiguous()
        desc.exponentials = exponentials.data_ptr()
        desc.exponentials_row_stride = exponentials.stride(0)
    else:
        if uniforms is None:
            raise ValueError("a sharded inverse-CDF draw needs the batch's uniforms on every slice")
        uniforms = uniforms.to(device=device, dtype=torch.float32).contiguous()
        if uniforms.shape != (rows,):
            raise ValueError("one uniform is required per row")
        desc.uniforms = uniforms.data_ptr()
        if masses is None:
            raise ValueError("a sharded inverse-CDF draw needs the masses gathered from every slice")
        ms = torch.stack(list(masses)) if isinstance(masses, (list, tuple)) else masses
        if ms.shape != (st.shape[0], rows) or ms.dtype != torch.int64:
            raise ValueError("masses must be the int64 [n_shards, rows] gathered from every slice")
        ms = ms.to(device).contiguous()
        d.masses = ms.data_ptr()
    picks = torch.empty(rows, _lib.FULL_PICK_BYTES // 8, dtype=torch.int64, device=device)
    d.sampler = _lib.ctypes.pointer(desc)
    d.out_picks = picks.data_ptr()
    lib = _lib.load()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_sampler_full_draw_run(_lib.ctypes.byref(d), stream)
    _lib.check(rc)
    return picks


def full_shard_finish(
    states,
    picks=None,
    *,
    vocab_size: int,
    draw: str = "inverse_cdf",
    uniforms: Optional[torch.Tensor] = None,
    check: bool = True,
) -> SampleResult:
    """Step 4 of a full-vocabulary draw over slices: the token from the gathered picks
    (``draw`` = ``"inverse_cdf"`` or ``"exponential_race"``) or, for ``"greedy"``, from the
    states alone, and its log-prob ``(z - M) - log S`` against the row's maximum and total.
    Returns what :func:`sample` returns for the unsharded logits; ``uniforms`` (inverse CDF)
    are checked and ``check`` raises as there."""
    modes = {"inverse_cdf": _lib.FULL_DRAW_CDF, "exponential_race": _lib.FULL_DRAW_RACE,
             "greedy": _lib.FULL_DRAW_GREEDY}
    if draw not in modes:
        raise ValueError("draw must be 'inverse_cdf', 'exponential_race' or 'greedy'")
    st = _gathered(states, _lib.FULL_STATE_BYTES // 8, "states")
    n_shards, rows, _ = st.shape
    device = st.device
    pk = None
    if draw != "greedy":
        if picks is None:
            raise ValueError("the draw's picks from every slice are required")
        pk = _gathered(picks, _lib.FULL_PICK_BYTES // 8, "picks").to(device)
        if pk.shape[:2] != (n_shards, rows):
            raise ValueError("picks must hold one pick per row of every slice")
    if draw == "inverse_cdf":
        if uniforms is None:
            raise ValueError("sampling requires one uniform per row")
        uniforms = uniforms.to(device=device, dtype=torch.float32).contiguous()
        if uniforms.shape != (rows,):
            raise ValueError("one uniform is required per row")
    ids = torch.empty(rows, dtype=torch.int64, device=device)
    lps = torch.empty(rows, dtype=torch.float32, device=device)
    kept = torch.empty(rows, dtype=torch.int32, device=device)
    status = torch.empty(rows, dtype=torch.int32, device=device)
    d = _lib.SamplerFullFinishDesc()
    d.struct_size = _lib.ctypes.sizeof(_lib.SamplerFullFinishDesc)
    d.rows, d.n_shards, d.draw = rows, n_shards, modes[draw]
    d.states = st.data_ptr()
    d.picks = _device_ptr(pk)
    d.uniforms = _device_ptr(uniforms if draw == "inverse_cdf" else None)
    d.vocab_size = vocab_size
    d.out_ids, d.out_logprob, d.out_kept, d.out_status = (ids.data_ptr(), lps.data_ptr(), kept.data_ptr(),
                                                          status.data_ptr())
    lib = _lib.load()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_sampler_full_finish_run(_lib.ctypes.byref(d), stream)
    _lib.check(rc)
    if check:
        if bool((status != 0).any()):
            _status_error(status)
    return SampleResult(ids, lps, kept, status)


def replay_log_probs(
    logits: torch.Tensor,
    token_ids: torch.Tensor,
    *,
    temperature: float = 1.0,
    history: Optional[torch.Tensor] = None,
    history_lens: Optional[torch.Tensor] = None,
    history_prompt_lens: Optional[torch.Tensor] = None,
    repetition_penalty: float = 1.0,
    presence_penalty: float = 0.0,
    frequency_penalty: float = 0.0,
    check: bool = True,
) -> torch.Tensor:
    """Processed log-prob of ``token_ids[r]`` under ``logits[r]`` for full-vocabulary sampling
    (the reference's training-eligible mode), bit for bit what :func:`sample` reported when it
    drew that token from the same logits with the same temperature and penalties, whichever
    draw it used.  This is the replay the reference requires to equal the behaviour log-prob
    exactly (``QwenPolicy.response_log_probs``, ``rl/qwen_policy.py:156-190``;
    ``cached_response_log_probs``, ``backends/qwen_kv_cache.py:117-132``).  Returns fp32
    ``[rows]``; with ``check`` raises the reference's ``ValueError`` for ids outside the
    vocabulary and for non-finite rows."""
    logits, history, history_lens = _rows_in(logits, history, history_lens, temperature, 0)
    rows = logits.shape[0]
    device = logits.device
    token_ids = torch.as_tensor(token_ids).to(device=device, dtype=torch.int64).reshape(-1).contiguous()
    if token_ids.shape != (rows,):
        raise ValueError("one token ID is required per row")
    ids = torch.empty(rows, dtype=torch.int64, device=device)
    lps = torch.empty(rows, dtype=torch.float32, device=device)
    status = torch.empty(rows, dtype=torch.int32, device=device)
    desc = _rows_desc(logits, history, history_lens, temperature, repetition_penalty, presence_penalty,
                      frequency_penalty, 0, 1.0, 0.0)
    plens = _prompt_lens(history_prompt_lens, history, logits.shape[0], logits.device)
    desc.history_prompt_lens = _device_ptr(plens)
    desc.replay_ids = token_ids.data_ptr()
    desc.out_ids, desc.out_logprob, desc.out_status = ids.data_ptr(), lps.data_ptr(), status.data_ptr()
    lib = _lib.load()
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.dsv41_sampler_run(_lib.ctypes.byref(desc), None, 0, stream)
    _lib.check(rc)
    if check:
        if bool((status != 0).any()):
            _status_error(status)
    return lps
