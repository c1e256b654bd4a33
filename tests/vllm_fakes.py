"""Stand-ins for the vLLM objects the connector's hooks read (vLLM is not installed).

Each carries exactly the attributes the reference's connector reads
(src/marathon/vllm_shift_connector.py): ``VllmConfig.cache_config.block_size``,
``.kv_transfer_config.kv_connector_extra_config``, ``.model_config.hf_text_config``;
``Request.request_id / kv_transfer_params / num_prompt_tokens``;
``SchedulerOutput.scheduled_new_reqs[i].req_id / block_ids / num_computed_tokens``,
``.scheduled_cached_reqs.req_ids / new_block_ids / num_computed_tokens``,
``.num_scheduled_tokens``, ``.finished_req_ids``; ``ForwardContext.no_compile_layers``
(layers with ``kv_cache``) and ``.virtual_engine``.  Block ids are given per KV-cache
group, as vLLM gives them.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from types import SimpleNamespace


def vllm_config(block_size=16, extra=None, head_dim=128, rope_theta=1e6,
                partial_rotary_factor=1.0):
    hf = SimpleNamespace(head_dim=head_dim, hidden_size=(head_dim or 128) * 32,
                         num_attention_heads=32,
                         rope_theta=rope_theta, partial_rotary_factor=partial_rotary_factor)
    return SimpleNamespace(
        cache_config=SimpleNamespace(block_size=block_size),
        kv_transfer_config=SimpleNamespace(kv_connector_extra_config=dict(extra or {})),
        model_config=SimpleNamespace(hf_text_config=hf),
    )


@dataclass
class Request:
    request_id: str
    kv_transfer_params: dict | None
    num_prompt_tokens: int


@dataclass
class NewRequestData:
    req_id: str
    block_ids: tuple  # per KV-cache group
    num_computed_tokens: int


@dataclass
class CachedRequestData:
    req_ids: list = field(default_factory=list)
    new_block_ids: list = field(default_factory=list)  # per request: per group, or None
    num_computed_tokens: list = field(default_factory=list)


@dataclass
class SchedulerOutput:
    scheduled_new_reqs: list = field(default_factory=list)
    scheduled_cached_reqs: CachedRequestData = field(default_factory=CachedRequestData)
    num_scheduled_tokens: dict = field(default_factory=dict)
    finished_req_ids: set = field(default_factory=set)


def step_output(new=(), cached=(), finished=()):
    """``new``: (rid, blocks, computed, scheduled); ``cached``: (rid, new blocks or None,
    computed, scheduled)."""
    out = SchedulerOutput(finished_req_ids=set(finished))
    for rid, blocks, computed, scheduled in new:
        out.scheduled_new_reqs.append(NewRequestData(rid, (list(blocks),), computed))
        out.num_scheduled_tokens[rid] = scheduled
    for rid, blocks, computed, scheduled in cached:
        c = out.scheduled_cached_reqs
        c.req_ids.append(rid)
        c.new_block_ids.append(None if blocks is None else (list(blocks),))
        c.num_computed_tokens.append(computed)
        out.num_scheduled_tokens[rid] = scheduled
    return out


def forward_context(kv_caches: dict, virtual_engine: int = 0, k_scales: dict | None = None):
    layers = {}
    for name, t in kv_caches.items():
        layer = SimpleNamespace(kv_cache=[t])
        if k_scales and name in k_scales:
            layer._k_scale_float = float(k_scales[name])
        layers[name] = layer
    layers["not_attention"] = SimpleNamespace()  # layers without a cache are skipped
    return SimpleNamespace(no_compile_layers=layers, virtual_engine=virtual_engine)
