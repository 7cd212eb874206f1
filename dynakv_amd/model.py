"""End-to-end Llama decoder over the compressed cache, and the same model with a dense cache.

The reference runs DynaKV inside HF's Llama (``custom_llama.py:93-323``, the attention module
``compressed_attention.py:204-386``) and times greedy generation with
``benchmark_throughput.py:17-82`` (tokens/s = batch * new tokens / wall time, prefill included).
This module is that model path for this build, written against the kernels directly (no
transformers model classes: their Cache API differs across versions, and the benchmark needs
only the forward math):

* ``RandomLlama``: Llama weights drawn on the device (N(0, 0.02) in bf16 by default) for a
  given shape (config 5: Llama-3-8B -- hidden 4096, 32 layers, 32/8 heads, head dim 128, FFN
  14336, vocab 128256), plus the DynaKV parameters per layer: a random orthogonal 128x128
  spectral basis per KV head for K and for V, the K/V projections merged with the basis
  transposes so that they emit coefficients (the one-time merge of
  ``compressed_attention.py:263-292``), and per-head cutoff heads whose bias ramps over the
  rank so that the retained fraction is close to a target (``retention``).
* ``CompressedLlama.generate``: prefill (cutoff head, packed append, reconstruct-and-attend)
  then greedy decode steps (cutoff head, decode append, routed decode attention). q/k/v and
  gate/up are one concatenated projection each; at decode sizes the projections run on the
  skinny GEMM (``kernels/model_ops.py``), with the residual add and the RMSNorm before them
  folded into its x staging for one or two rows, and the SwiGLU product is one kernel --
  the same stages serve the dense baseline.
* ``DenseLlama.generate``: the uncompressed-cache baseline of the same weights (K/V kept in
  full in a preallocated cache; decode attention by the same split kernel over that cache read
  as a packed cache with all 128 dims per token and an identity basis, prefill attention by
  torch's scaled_dot_product_attention).
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from .formats import merge_projection
from .kernels.compressed_cache import CustomDynamicCache
from .kernels.cutoff import CutoffHead
from .kernels.decode import dense_append_, dense_decode_attention, grouped_decode_attention
from .kernels.layer import DecodeLayerPlan
from .kernels.model_ops import linear, rmsnorm_glu, rmsnorm_linear
from .kernels.prefill import coef_prefill_attention, rope_dense_
from .kernels.router import KernelPolicy


@dataclass(frozen=True)
class LlamaShape:
    hidden: int = 4096
    layers: int = 32
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 128256
    theta: float = 500000.0
    eps: float = 1e-5


@dataclass
class LayerWeights:
    ln1: torch.Tensor
    w_qkv_c: torch.Tensor  # (H + 2 G Dh, H): q, then the merged K / V coefficient projections
    w_qkv: torch.Tensor    # (H + 2 G Dh, H): q, K, V of the dense baseline
    wq: torch.Tensor       # views of w_qkv_c (wq, wk_c, wv_c) and of w_qkv (wk, wv)
    wk: torch.Tensor       # dense K projection (the baseline)
    wv: torch.Tensor
    wk_c: torch.Tensor     # merged: emits per-head K coefficients
    wv_c: torch.Tensor
    wo: torch.Tensor
    ln2: torch.Tensor
    w_gu: torch.Tensor     # (2 * ffn, hidden): gate and up rows interleaved (2j gate, 2j+1 up)
    w_gate: torch.Tensor   # views of w_gu
    w_up: torch.Tensor
    w_down: torch.Tensor
    k_basis: torch.Tensor  # (G, R, Dh) rank-major
    v_basis: torch.Tensor
    cutoff: CutoffHead = field(repr=False)


def _orthogonal(n: int, count: int, gen: torch.Generator, device) -> torch.Tensor:
    a = torch.randn(count, n, n, generator=gen, device=device, dtype=torch.float32)
    q, r = torch.linalg.qr(a)
    return q * torch.sign(torch.diagonal(r, dim1=-2, dim2=-1)).unsqueeze(-2)


def ramp_for_retention(D: int, retention: float) -> float:
    """Slope beta of the cutoff bias beta * j / D for which flip(cumsum(softmax)) >= 0.1 keeps
    ``retention * D`` dims when the input term is small: the mass below index D * (1 - r) is
    0.1, i.e. (e^{beta (1-r)} - 1) / (e^{beta} - 1) = 0.1, solved by bisection."""
    lo, hi = 1e-3, 60.0
    target_m = 1.0 - retention
    for _ in range(100):
        mid = 0.5 * (lo + hi)
        frac = math.expm1(mid * target_m) / math.expm1(mid)
        if frac > 0.1:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


class RandomLlama:
    def __init__(self, shape: LlamaShape = LlamaShape(), *, device="cuda", dtype=torch.bfloat16,
                 seed: int = 0, retention: float = 0.47, std: float = 0.02):
        self.shape = shape
        self.dtype = dtype
        self.device = torch.device(device)
        g = torch.Generator(device=self.device)
        g.manual_seed(seed)
        s = shape
        H, Dh, G = s.hidden, s.head_dim, s.kv_heads

        def rnd(*dims):
            return (torch.randn(*dims, generator=g, device=self.device, dtype=torch.float32)
                    * std).to(dtype)

        self.embed = rnd(s.vocab, H)
        self.norm = torch.ones(H, device=self.device, dtype=dtype)
        self.lm_head = rnd(s.vocab, H)
        beta = ramp_for_retention(Dh, retention)
        ramp = (beta * torch.arange(Dh, device=self.device, dtype=torch.float32) / Dh).to(dtype)
        self.layers = []
        for _ in range(s.layers):
            wk, wv = rnd(G * Dh, H), rnd(G * Dh, H)
            Uk = _orthogonal(Dh, G, g, self.device)  # (G, d, r): K_g = U_g c_g
            Uv = _orthogonal(Dh, G, g, self.device)
            # coefficients c_g = U_g^T k_g: the projection merged with the basis transpose (the
            # reference's one-time merge, k_proj <- k_down @ k_proj, per KV group)
            wk_c = merge_projection(wk.float().view(G, Dh, H), Uk.transpose(1, 2))[0]
            wv_c = merge_projection(wv.float().view(G, Dh, H), Uv.transpose(1, 2))[0]
            wk_c, wv_c = wk_c.reshape(G * Dh, H), wv_c.reshape(G * Dh, H)
            cut = [rnd(G, Dh, Dh) for _ in range(2)]
            bias = [ramp.expand(G, Dh).contiguous() for _ in range(2)]
            w_gu = rnd(2 * s.ffn, H)
            wq = rnd(H, H)
            w_qkv_c = torch.cat([wq, wk_c.to(dtype), wv_c.to(dtype)])
            w_qkv = torch.cat([wq, wk, wv])
            GD = G * Dh
            self.layers.append(LayerWeights(
                ln1=torch.ones(H, device=self.device, dtype=dtype), w_qkv_c=w_qkv_c, w_qkv=w_qkv,
                wq=w_qkv_c[:H], wk=w_qkv[H:H + GD], wv=w_qkv[H + GD:],
                wk_c=w_qkv_c[H:H + GD], wv_c=w_qkv_c[H + GD:], wo=rnd(H, H),
                ln2=torch.ones(H, device=self.device, dtype=dtype),
                w_gu=w_gu, w_gate=w_gu[0::2], w_up=w_gu[1::2], w_down=rnd(H, s.ffn),
                k_basis=Uk.transpose(1, 2).contiguous().to(dtype),
                v_basis=Uv.transpose(1, 2).contiguous().to(dtype),
                cutoff=CutoffHead(cut[0], bias[0], cut[1], bias[1], groups=G)))




def _rope_q(q: torch.Tensor, pos0: int, theta: float) -> torch.Tensor:
    """q (B, S, Hq, Dh) -> rotated (B, Hq, S, Dh) contiguous."""
    qh = q.transpose(1, 2).contiguous()
    return rope_dense_(qh, theta=theta, pos0=pos0)


class _Generator:
    def __init__(self, model: RandomLlama):
        self.m = model
        self.s = model.shape

    def _split(self, y: torch.Tensor):
        """The q, K and V column ranges of a fused projection output (views)."""
        H, GD = self.s.hidden, self.s.kv_heads * self.s.head_dim
        return y[..., :H], y[..., H:H + GD], y[..., H + GD:]

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        return rmsnorm_linear(x, None, self.m.norm, self.s.eps, self.m.lm_head)[0]

    def _run(self, x: torch.Tensor, attn, qkv: str) -> torch.Tensor:
        """The decoder layers over the residual stream ``x`` (B, S, hidden); returns the final
        residual stream. ``attn(i, lw, y)`` takes layer i's q/k/v projection output ``y``
        (weight ``getattr(lw, qkv)``) and returns its attention output (B, S, hidden) before the
        output projection. Each residual add and the norm after it are fused into the
        projection that consumes them (decode), or one kernel before it (prefill)."""
        eps = self.s.eps
        delta = None
        for i, lw in enumerate(self.m.layers):
            y, x = rmsnorm_linear(x, delta, lw.ln1, eps, getattr(lw, qkv))
            h, x = rmsnorm_glu(x, linear(attn(i, lw, y), lw.wo), lw.ln2, eps, lw.w_gu)
            delta = linear(h, lw.w_down)
        return x + delta

    def generate(self, prompt: torch.Tensor, new_tokens: int) -> dict:
        """Greedy decode; returns tokens, timings and cache bytes."""
        torch.cuda.synchronize(self.m.device)
        t0 = time.perf_counter()
        x = self.prefill(prompt)
        tok = self.logits(x[:, -1:]).argmax(-1)  # (B, 1)
        out = [tok]
        torch.cuda.synchronize(self.m.device)
        t1 = time.perf_counter()
        pos = prompt.shape[1]
        for _ in range(new_tokens - 1):
            x = self.decode(tok, pos)
            tok = self.logits(x).argmax(-1)
            out.append(tok)
            pos += 1
        torch.cuda.synchronize(self.m.device)
        t2 = time.perf_counter()
        B = prompt.shape[0]
        return {
            "tokens": torch.cat(out, dim=1),
            "prefill_s": t1 - t0,
            "decode_s": t2 - t1,
            "tokens_per_s": B * new_tokens / (t2 - t0),
            "decode_tokens_per_s": B * (new_tokens - 1) / max(t2 - t1, 1e-9),
            "kv_bytes": self.kv_bytes(),
        }


class CompressedLlama(_Generator):
    """The model over DynaKV's packed cache (per-head layout, rows b*G + g)."""

    def __init__(self, model: RandomLlama, policy: KernelPolicy | None = None,
                 one_call_layers: bool = True):
        super().__init__(model)
        self.policy = policy or KernelPolicy()
        self.cache = CustomDynamicCache()
        self.one_call_layers = one_call_layers
        self.plans: dict = {}

    def _qkv(self, lw, h):
        """``h``: the layer's fused q/k/v projection output (B, S, H + 2 G Dh)."""
        B, S, _ = h.shape
        s = self.s
        q, kc, vc = self._split(h)
        q = q.reshape(B, S, s.heads, s.head_dim)
        kc, vc = kc.contiguous(), vc.contiguous()  # (B, S, G*Dh) coefficients
        k_out, v_out, len_k, len_v, _, _ = lw.cutoff.kv_process_fused(kc, vc)
        G, Dh = s.kv_heads, s.head_dim
        if B == 1:
            # rows b*G + g are strided views (row stride Dh, token stride G*Dh): the appends and
            # the prefill products take the strides, so no transposed copy is made
            rows_k = k_out.view(S, G, Dh).transpose(0, 1)
            rows_v = v_out.view(S, G, Dh).transpose(0, 1)
            lk = len_k.view(S, G).transpose(0, 1)
            lv = len_v.view(S, G).transpose(0, 1)
            return q, rows_k, lk, rows_v, lv
        rows_k = k_out.view(B, S, G, Dh).transpose(1, 2).reshape(B * G, S, Dh)
        rows_v = v_out.view(B, S, G, Dh).transpose(1, 2).reshape(B * G, S, Dh)
        lk = len_k.view(B, S, G).transpose(1, 2).reshape(B * G, S).contiguous()
        lv = len_v.view(B, S, G).transpose(1, 2).reshape(B * G, S).contiguous()
        return q, rows_k, lk, rows_v, lv

    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        s = self.s
        self.cache.reset()
        self.plans = {}
        x = F.embedding(prompt, self.m.embed)
        B, S = prompt.shape

        pending = []

        def attn(i, lw, y):
            q, rk, lk, rv, lv = self._qkv(lw, y)
            pending.append((i, rk, lk, rv, lv))
            qh = _rope_q(q, 0, s.theta)
            # the masked coefficients are what the packed cache returns once appended
            a = coef_prefill_attention(qh, rk, rv, lw.k_basis, lw.v_basis, theta=s.theta)
            return a.transpose(1, 2).reshape(B, S, s.hidden)

        x = self._run(x, attn, "w_qkv_c")
        # every layer's appends after the forward pass: one host synchronisation in all
        self.cache.update_sp_prefill_many(pending, s.head_dim)
        return x

    def decode(self, tok: torch.Tensor, pos: int) -> torch.Tensor:
        s = self.s
        x = F.embedding(tok, self.m.embed)  # (B, 1, H)
        B = tok.shape[0]

        def attn(i, lw, y):
            plan = self.plans.get(i)
            if plan is not None and plan.can_step():
                # one call: cutoff head, K+V append, q RoPE, routed attention
                # one projection; q and the coefficients are views into its output
                q, kc, vc = self._split(y.view(B, -1))
                a = plan.step(q.view(B, s.heads, s.head_dim), kc, vc, pos)
            else:
                q, rk, lk, rv, lv = self._qkv(lw, y)
                fk, fv, tk, tv, ok, ov = self.cache.update_sp(rk, lk, rv, lv, s.head_dim, i,
                                                              s.head_dim)
                L = self.cache.get_seq_length_sp(i)
                qh = _rope_q(q, pos, s.theta)[:, :, 0]  # (B, Hq, Dh)
                a = grouped_decode_attention(qh, fk, fv, tk, ok, tv, ov, lw.k_basis, lw.v_basis,
                                             theta=s.theta, route=self.policy.select(L))
                if self.one_call_layers:
                    self.plans[i] = DecodeLayerPlan(self.cache, i, lw.cutoff, lw.k_basis,
                                                    lw.v_basis, batch=B, heads=s.heads,
                                                    theta=s.theta, policy=self.policy)
            return a.reshape(B, 1, s.hidden)

        return self._run(x, attn, "w_qkv_c")

    def kv_bytes(self) -> int:
        """Stored bytes of the packed caches: the used part of each row plus 8 bytes of
        lengths/offsets per token and row."""
        tot = 0
        for slots in (self.cache.key_cache_sp, self.cache.value_cache_sp):
            for c in slots:
                if c is None:
                    continue
                flat, lens, offs, ptr, seq = c[0], c[1], c[2], c[3], c[4]
                tot += int(ptr.sum()) * flat.element_size() + 8 * lens.shape[0] * seq
        return tot


# torch's fused attention kernels only: an input they do not take raises instead of running the
# composite (math) path
_FAST_SDPA = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]


class DenseLlama(_Generator):
    """The same weights with an uncompressed cache, the reference's baseline (the original model
    with transformers' KV cache, ``scripts/benchmark_throughput.py:17-77``): every token's
    rotated key and its value kept in full (head dim 128 per KV head). A decode step writes the
    new token's rotated key and value and rotates q in one launch (``dkv_dense_append``), then
    runs dense GQA decode attention (``dkv_decode_dense``: no reconstruction, no RoPE in the
    attention, fp32 scores). Prefill attention is torch's fused attention on the rotated keys."""

    def __init__(self, model: RandomLlama, max_len: int = 4096, attention: str = "kernel"):
        """``attention``: "kernel" (``dkv_decode_dense``) or "sdpa" (torch's
        ``scaled_dot_product_attention`` over the cached keys and values, the attention path the
        reference's uncompressed transformers model takes)."""
        super().__init__(model)
        if attention not in ("kernel", "sdpa"):
            raise ValueError("attention must be 'kernel' or 'sdpa'")
        self.max_len = max_len
        self.attention = attention
        self.k = self.v = None
        self.len = 0

    def _kv(self, lw, y, pos0):
        """``y``: the layer's fused q/k/v projection output (B, S, H + 2 G Dh). Returns the
        rotated q (B, Hq, S, Dh) and K (before RoPE) / V as (B, G, S, Dh)."""
        B, S, _ = y.shape
        s = self.s
        q, k, v = self._split(y)
        q = q.reshape(B, S, s.heads, s.head_dim)
        k = k.reshape(B, S, s.kv_heads, s.head_dim).transpose(1, 2)
        v = v.reshape(B, S, s.kv_heads, s.head_dim).transpose(1, 2)
        return _rope_q(q, pos0, s.theta), k, v

    def prefill(self, prompt: torch.Tensor) -> torch.Tensor:
        s = self.s
        B, S = prompt.shape
        dev, dt = self.m.device, self.m.dtype
        G, Dh = s.kv_heads, s.head_dim
        rows = B * G
        # per layer: K and V rows (b*G + g) of max_len tokens x Dh, tokens back to back, and the
        # shared tables of the packed view (128 dims per token, token t at offset 128 t)
        self.k = [torch.empty((rows, self.max_len * Dh), device=dev, dtype=dt)
                  for _ in range(s.layers)]
        self.v = [torch.empty((rows, self.max_len * Dh), device=dev, dtype=dt)
                  for _ in range(s.layers)]
        hpg = s.heads // s.kv_heads
        x = F.embedding(prompt, self.m.embed)

        def attn(i, lw, y):
            qh, k, v = self._kv(lw, y, 0)
            kr = rope_dense_(k.contiguous(), theta=s.theta, pos0=0)
            self.k[i][:, :S * Dh] = kr.reshape(rows, S * Dh)
            self.v[i][:, :S * Dh] = v.reshape(rows, S * Dh)
            with sdpa_kernel(_FAST_SDPA):
                a = F.scaled_dot_product_attention(qh, kr.repeat_interleave(hpg, dim=1),
                                                   v.repeat_interleave(hpg, dim=1),
                                                   is_causal=True)
            return a.transpose(1, 2).reshape(B, S, s.hidden)

        x = self._run(x, attn, "w_qkv")
        self.len = S
        return x

    def decode(self, tok: torch.Tensor, pos: int) -> torch.Tensor:
        """One token: the rotated K and V written at position len (q rotated at ``pos`` in the
        same launch), then dense decode attention over len + 1 tokens."""
        s = self.s
        x = F.embedding(tok, self.m.embed)
        B = tok.shape[0]
        L = self.len
        Dh = s.head_dim

        def attn(i, lw, y):
            y2 = y[:, 0, :]
            dense_append_(y2, self.k[i], self.v[i], q_pos=pos, k_pos=L, heads=s.heads,
                          kv_heads=s.kv_heads, theta=s.theta)
            qh = y2[:, :s.heads * Dh].view(B, s.heads, Dh)
            if self.attention == "sdpa":
                G, hpg = s.kv_heads, s.heads // s.kv_heads
                kk = self.k[i][:, :(L + 1) * Dh].view(B, G, L + 1, Dh)
                vv = self.v[i][:, :(L + 1) * Dh].view(B, G, L + 1, Dh)
                with sdpa_kernel(_FAST_SDPA):
                    a = F.scaled_dot_product_attention(
                        qh.unsqueeze(2), kk.repeat_interleave(hpg, dim=1),
                        vv.repeat_interleave(hpg, dim=1))
                return a.reshape(B, 1, s.hidden)
            a = dense_decode_attention(qh, self.k[i], self.v[i], L + 1)
            return a.reshape(B, 1, s.hidden)

        x = self._run(x, attn, "w_qkv")
        self.len = L + 1
        return x

    def kv_bytes(self) -> int:
        """Stored K and V payload: every token of every (batch, KV head) row at 128 dims."""
        s = self.s
        rows = self.k[0].shape[0] if self.k else 0
        return 2 * s.layers * rows * self.len * s.head_dim * self.m.embed.element_size()
