"""Model-level drift check: a plain f32 Qwen3 forward from the unquantised
checkpoint (tools/fp32_ref.py:28-119), sharing nothing with the int8 path
(no quantisation, no 32-key blocks, no online softmax), and the statistics
that compare the W8A8 device logits with it.

The forward follows fp32_ref.py: RMSNorm in f64 then f32 (hidden, and per
head for q/k), rotate-half RoPE with f32 tables of f64 angles, causal
softmax attention with grouped KV heads, SwiGLU MLP, final norm, lm_head
(the embedding when tied).  It runs in torch f32 on the device when one is
present (the products stay f32 and contiguous), else on the CPU.

    python -m q3ops.fp32_ref --model-dir DIR --ids 151644,9707 [--compare]
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path

import numpy as np

__all__ = ["F32Model", "drift_stats", "compare_device", "main"]


class F32Model:
    def __init__(self, model_dir: str | Path, device: str | None = None, layers: int = 0):
        import torch
        from safetensors import safe_open
        model_dir = Path(model_dir)
        self.cfg = json.loads((model_dir / "config.json").read_text())
        c = self.cfg
        self.hidden = int(c["hidden_size"])
        self.heads, self.kv_heads = int(c["num_attention_heads"]), int(c["num_key_value_heads"])
        self.head_dim, self.inter = int(c["head_dim"]), int(c["intermediate_size"])
        self.layers = int(layers or c["num_hidden_layers"])
        self.eps = float(c.get("rms_norm_eps", 1e-6))
        self.theta = float(c.get("rope_theta", 1e6))
        self.device = device or ("cuda" if torch.cuda.is_available() else "cpu")
        f = safe_open(str(model_dir / "model.safetensors"), framework="pt")

        def t(name):
            return f.get_tensor(name).to(device=self.device, dtype=torch.float32).contiguous()

        self.emb = t("model.embed_tokens.weight")
        self.lm = t("lm_head.weight") if "lm_head.weight" in set(f.keys()) else self.emb
        self.nf = t("model.norm.weight")
        self.w = []
        for li in range(self.layers):
            p = f"model.layers.{li}."
            self.w.append({k: t(p + k + ".weight") for k in (
                "input_layernorm", "post_attention_layernorm", "self_attn.q_norm",
                "self_attn.k_norm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")})
        self.rope_sign = 1.0  # tests plant a mistake by flipping it

    def rmsnorm(self, x, w):
        import torch
        xd = x.to(torch.float64)
        var = (xd * xd).mean(dim=-1, keepdim=True)
        return (xd / torch.sqrt(var + self.eps) * w.to(torch.float64)).to(torch.float32)

    def forward(self, ids) -> np.ndarray:
        """Logits [len(ids)][vocab] (f32) for the prompt ids at positions 0..n-1."""
        import torch
        n, hd, half = len(ids), self.head_dim, self.head_dim // 2
        dev = self.device
        x = self.emb[torch.as_tensor(list(ids), device=dev, dtype=torch.long)]
        inv = 1.0 / (self.theta ** (torch.arange(half, dtype=torch.float64) / half))
        ang = torch.arange(n, dtype=torch.float64)[:, None] * inv[None, :]
        cos = torch.cos(ang).to(torch.float32).to(dev)[:, None, :]
        sin = (self.rope_sign * torch.sin(ang)).to(torch.float32).to(dev)[:, None, :]
        mask = torch.triu(torch.ones(n, n, dtype=torch.bool, device=dev), diagonal=1)
        group = self.heads // self.kv_heads

        def rope(t):
            a, b = t[..., :half], t[..., half:]
            return torch.cat([a * cos - b * sin, a * sin + b * cos], dim=-1)

        for w in self.w:
            h = self.rmsnorm(x, w["input_layernorm"])
            q = (h @ w["self_attn.q_proj"].T).reshape(n, self.heads, hd)
            k = (h @ w["self_attn.k_proj"].T).reshape(n, self.kv_heads, hd)
            v = (h @ w["self_attn.v_proj"].T).reshape(n, self.kv_heads, hd)
            q = rope(self.rmsnorm(q, w["self_attn.q_norm"]))
            k = rope(self.rmsnorm(k, w["self_attn.k_norm"]))
            qh = q.transpose(0, 1).contiguous()                                  # [heads][n][hd]
            kt = k.repeat_interleave(group, dim=1).permute(1, 2, 0).contiguous()  # [heads][hd][n]
            vh = v.repeat_interleave(group, dim=1).transpose(0, 1).contiguous()  # [heads][n][hd]
            s = torch.bmm(qh, kt) * (1.0 / float(np.sqrt(hd)))
            s = s.masked_fill(mask[None], float("-inf"))
            s = s - s.max(dim=-1, keepdim=True).values
            pr = torch.exp(s)
            pr = pr / pr.sum(dim=-1, keepdim=True)
            attn = torch.bmm(pr, vh).transpose(0, 1).reshape(n, self.heads * hd)
            x = x + attn @ w["self_attn.o_proj"].T
            h = self.rmsnorm(x, w["post_attention_layernorm"])
            g = h @ w["mlp.gate_proj"].T
            u = h @ w["mlp.up_proj"].T
            x = x + ((g / (1.0 + torch.exp(-g))) * u) @ w["mlp.down_proj"].T
        return (self.rmsnorm(x, self.nf) @ self.lm.T).cpu().numpy()


def drift_stats(ref: np.ndarray, got: np.ndarray) -> dict:
    """How far got (W8A8) is from ref (f32), one logits row."""
    r, g = np.asarray(ref, np.float64).ravel(), np.asarray(got, np.float64).ravel()
    d = g - r
    top5r, top5g = set(np.argsort(-r)[:5].tolist()), set(np.argsort(-g)[:5].tolist())
    return {"max_abs": float(np.max(np.abs(d))),
            "rel_l2": float(np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30)),
            "cosine": float(r @ g / max(np.linalg.norm(r) * np.linalg.norm(g), 1e-30)),
            "top1_equal": int(np.argmax(r)) == int(np.argmax(g)),
            "top5_overlap": len(top5r & top5g)}


def compare_device(model_dir: str | Path, ids, max_seq: int = 256) -> dict:
    """Converts the checkpoint, runs the prompt through the device model in
    one chunk (logits of the last row) and compares with the f32 model."""
    from .convert import convert
    from .model import LM_LOGITS, Model
    n = len(ids)
    lay, blob = convert(model_dir, seq=max(32, n), max_seq=max(max_seq, n), n_prompt=n,
                        ids=",".join(str(int(t)) for t in ids))
    m = Model(lay, np.ascontiguousarray(blob))
    try:
        m.forward_chunk(0, n, LM_LOGITS, optimize_tail=True)
        got = m.stage("logits", 1)[0].copy()
    finally:
        m.close()
    ref = F32Model(model_dir).forward(ids)[-1]
    return drift_stats(ref, got)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="f32 Qwen3 forward and W8A8 drift")
    ap.add_argument("--model-dir", required=True)
    ap.add_argument("--ids", required=True, help="comma-separated prompt ids")
    ap.add_argument("--compare", action="store_true", help="also run the W8A8 device model")
    a = ap.parse_args(argv)
    ids = [int(t) for t in a.ids.split(",") if t.strip()]
    last = F32Model(a.model_dir).forward(ids)[-1]
    top = np.argsort(-last)[:5]
    print("f32 top-5:", [(int(i), float(last[i])) for i in top])
    if a.compare:
        print("W8A8 drift:", json.dumps(compare_device(a.model_dir, ids)))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
