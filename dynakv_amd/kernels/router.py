"""Runtime routing between the short (fused) and long (two-stage) decode kernels.

Same surface and behaviour as the reference ``src/dynakv/kernels/router.py:8-59``:
``KernelPolicy(switch_tokens=500).select(L)`` returns ``"short_fused"`` for ``L < switch_tokens``
and ``"long_two_stage"`` otherwise, raising ``ValueError`` for negative lengths; the caller passes
the post-append cache length. Both routes run on the gfx950 split-K kernel when the inputs fit it
(f16/bf16, head dim 128, rank <= 128, a basis shared per query-head group), with the route's own
semantics (masking value, score rounding, denominator clamp); otherwise the reference-semantics
vector kernels run.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class KernelPolicy:
    """Select the fused kernel below ``switch_tokens`` and two-stage at or above it."""

    switch_tokens: int = 500

    def select(self, cache_length: int) -> str:
        if cache_length < 0:
            raise ValueError("cache_length must be non-negative")
        return "short_fused" if cache_length < self.switch_tokens else "long_two_stage"


def compressed_decode_attention(
    *, q, k_flat, k_up, v_flat, v_up, key_lengths, key_offsets,
    value_lengths, value_offsets, theta: float, cache_length: int,
    policy: KernelPolicy | None = None,
):
    """Decode attention over the packed cache, routed on ``cache_length``.

    Arguments follow the reference (``router.py:20-24``): ``q`` is ``(B, Hq, 1, Dh)`` already
    RoPE'd at the current position, ``k_flat``/``v_flat`` are ``(B, cap)`` packed rows,
    ``k_up``/``v_up`` are ``(Hb, R, Dh)`` bases (``Hb`` divides ``Hq``), the length/offset tables
    are ``(B, S)`` int32 views. Returns ``(B, Hq, Dh)`` in ``q``'s dtype.
    """
    policy = policy or KernelPolicy()
    selected = policy.select(cache_length)
    if selected == "short_fused":
        from .fused import fused_attention_dispatch

        return fused_attention_dispatch(
            q=q, k_flat=k_flat, k_up=k_up, v_flat=v_flat, v_up=v_up,
            l_k=key_lengths, o_k=key_offsets, l_v=value_lengths, o_v=value_offsets,
            theta=theta,
        )

    from .two_stage import two_stage_attention

    return two_stage_attention(
        q=q, k_flat=k_flat, k_up=k_up, v_flat=v_flat, v_up=v_up,
        key_lengths=key_lengths, key_offsets=key_offsets,
        value_lengths=value_lengths, value_offsets=value_offsets, theta=theta,
    )
