"""Score modifications (absent from the reference; FlexAttention's ``score_mod``).

A score mod rewrites the scaled logit ``s = scale * q.k`` before masking.
The MI355X kernels support a fixed, fused set, applied in this order:

1. ALiBi bias: ``s += slope[h] * (kv_idx - q_idx)``
2. tanh soft-cap: ``s = cap * tanh(s / cap)``

:class:`ScoreSpec` objects are callable with PyTorch's signature
``score_mod(score, b, h, q_idx, kv_idx)`` on numpy arrays or torch tensors,
so the same object drives the GPU kernels and host-side checks.
"""
from typing import Optional

import numpy as np


def _is_torch(x):
    return type(x).__module__.startswith("torch")


def alibi_slopes(num_heads: int) -> np.ndarray:
    """ALiBi slopes ``2 ** (-8 * h / num_heads)`` for 0-based head index h
    (head 0 has slope 1)."""
    h = np.arange(num_heads, dtype=np.float64)
    return (2.0 ** (-8.0 * h / num_heads)).astype(np.float32)


class ScoreSpec:
    """Fused score modification: optional ALiBi slopes (per q head) then an
    optional tanh soft-cap."""

    def __init__(self, alibi: Optional[np.ndarray] = None, softcap: float = 0.0):
        self.alibi = None if alibi is None else np.ascontiguousarray(alibi, dtype=np.float32).reshape(-1)
        self.softcap = float(softcap or 0.0)
        if self.softcap < 0:
            raise ValueError("softcap must be positive")
        self._torch_slopes = {}

    def key(self):
        return ("ScoreSpec", None if self.alibi is None else self.alibi.tobytes(), self.softcap)

    def device_slopes(self, device):
        """The ALiBi slopes as a float32 tensor on ``device`` (cached)."""
        import torch
        dev = torch.device(device)
        if dev not in self._torch_slopes:
            self._torch_slopes[dev] = torch.as_tensor(self.alibi, device=dev)
        return self._torch_slopes[dev]

    def __eq__(self, other):
        return isinstance(other, ScoreSpec) and self.key() == other.key()

    def __hash__(self):
        return hash(self.key())

    def __repr__(self):
        parts = []
        if self.alibi is not None:
            parts.append(f"alibi[{len(self.alibi)}]")
        if self.softcap > 0:
            parts.append(f"softcap({self.softcap:g})")
        return "ScoreSpec(" + ", ".join(parts) + ")"

    def then(self, other: "ScoreSpec") -> "ScoreSpec":
        """Compose: apply ``self`` then ``other`` (must keep the order ALiBi -> soft-cap)."""
        if self.softcap > 0 and other.alibi is not None:
            raise NotImplementedError("the fused epilogue applies ALiBi before the soft-cap")
        if self.alibi is not None and other.alibi is not None:
            raise NotImplementedError("only one ALiBi term is supported")
        if self.softcap > 0 and other.softcap > 0:
            raise NotImplementedError("only one soft-cap is supported")
        return ScoreSpec(self.alibi if self.alibi is not None else other.alibi,
                         self.softcap if self.softcap > 0 else other.softcap)

    def __call__(self, score, b, h, q_idx, kv_idx):
        s = score
        if type(s).__name__ == "Sym":  # traced as part of a callable lowered onto the kernels
            import torch
            if self.alibi is not None:
                if "cpu" not in self._torch_slopes:
                    self._torch_slopes["cpu"] = torch.from_numpy(self.alibi)
                s = s + self._torch_slopes["cpu"][h] * (kv_idx - q_idx)
            if self.softcap > 0:
                s = self.softcap * torch.tanh(s / self.softcap)
            return s
        if self.alibi is not None:
            if _is_torch(s):
                import torch
                dev = s.device
                if dev not in self._torch_slopes:
                    self._torch_slopes[dev] = torch.as_tensor(self.alibi, device=dev)
                slope = self._torch_slopes[dev][h]
                s = s + slope * (kv_idx - q_idx).to(s.dtype)
            else:
                s = s + self.alibi[h] * np.asarray(kv_idx - q_idx, dtype=np.asarray(s).dtype)
        if self.softcap > 0:
            if _is_torch(s):
                import torch
                s = self.softcap * torch.tanh(s / self.softcap)
            else:
                s = self.softcap * np.tanh(s / self.softcap)
        return s


def alibi_score_mod(num_heads_or_slopes) -> ScoreSpec:
    """ALiBi bias.  Pass the number of query heads (slopes ``2**(-8h/H)``) or an
    explicit slope per head."""
    if np.ndim(num_heads_or_slopes) == 0:
        return ScoreSpec(alibi=alibi_slopes(int(num_heads_or_slopes)))
    return ScoreSpec(alibi=np.asarray(num_heads_or_slopes, dtype=np.float32))


def softcap_score_mod(cap: float) -> ScoreSpec:
    """tanh soft-cap ``s -> cap * tanh(s / cap)``."""
    return ScoreSpec(softcap=cap)


def compose_score_mods(*mods: ScoreSpec) -> ScoreSpec:
    """Apply the given score mods in order (ALiBi must precede the soft-cap)."""
    out = ScoreSpec()
    for m in mods:
        out = out.then(m)
    return out
