"""dsv41_rocm — MI355X (gfx950) token sampler and fused selected-token log-prob.

Drop-in for Tiny-DSV41's rollout sampling step (``dsv41_train/rl/rollout.py:144-150``), its
selected-token log-prob head (``dsv41_train/models/dsv4/model.py:679-684``,
``dsv41_train/rl/native_lora.py:80-82``) with its backward, and the decoupled Token-TIS loss
(``dsv41_train/rl/algorithm.py:249-346``), backed by hand-written HIP kernels in
``libdsv41hip.so`` (C ABI: ``include/dsv41_rocm.h``).
"""

from ._lib import load as load_library  # noqa: F401
from .logprob import combine_states, score_targets, selected_log_probs, shard_states, token_log_probs  # noqa: F401
from .ops import sample_rows, selected_log_probs_op  # noqa: F401  (registers torch.ops.dsv41_rocm)
from .sampling import (SampleResult, ShardCandidates, full_shard_draw, full_shard_finish, full_shard_masses,  # noqa: F401
                       full_shard_states, merge_shards, replay_log_probs, sample, sample_next, sample_shard,
                       validate_temperature)
from .rollout import generate_group_responses, generate_response  # noqa: F401
from .tis import decoupled_token_tis_loss, grpo_loss  # noqa: F401

__all__ = ["SampleResult", "sample", "sample_next", "validate_temperature", "load_library",
           "ShardCandidates", "sample_shard", "merge_shards", "replay_log_probs",
           "full_shard_states", "full_shard_masses", "full_shard_draw", "full_shard_finish",
           "selected_log_probs", "score_targets", "token_log_probs", "shard_states", "combine_states", "sample_rows", "selected_log_probs_op",
           "decoupled_token_tis_loss", "grpo_loss", "generate_response", "generate_group_responses"]
