"""Staged CPU reference of the SmolLM decoder -- TEST INFRASTRUCTURE ONLY.

Restates FrozenSmolLayer.reference_cpu (reference torch_npu_smollm.py:142-193) and
FrozenSmolIO (torch_npu_smollm_io.py:45-61) in torch on the CPU, with the RoPE base and
the KV capacity as parameters (the reference fixes theta=1e5 and 64 slots, :111-116).
Every fp16 rounding point of the reference is kept:

  linear     W8 per-row: fp16(x_f64 . (q*s)_f64^T); 4-bit: fp16(x_f32 . dequant_f32^T);
             protected: fp16(x_f32 . W16_f32^T); correction z = fp16(x.V^T),
             d = fp16(z.U^T), y = fp16(y + d)                         (:150-165)
  RMSNorm    fp16(fp16(x * rsqrt(mean(x^2) + 1e-5)) * gamma)          (:166-168)
  RoPE       fp16 cos/sin tables; fp16(fp16(v*cos) + fp16(rot(v)*sin)) (:113-116, :174-177)
  attention  scores fp16(q.k^T), fp16(* 0.125), causal -inf, softmax fp32 -> fp16,
             P.V fp32 -> fp16; GQA 3 -> 9 by repeat_interleave       (:178-182)
  MLP        fp16(silu(gate_f32)) * up -> fp16                        (:188-190)
  logits     fp16(fp32 RMS) * gamma, then F.linear with the tied fp16 embedding (io :57-61)

The decode step is the KV-cached row of the same computation: at position p it reads
keys/values 0..p and uses the RoPE row p.  Pinning (tests/test_smollm_cpu.py): the attention
outputs and logits of a full forward agree with transformers' LlamaForCausalLM (fp32, eager
attention, built offline from a local LlamaConfig and loaded with this oracle's effective
weights) within 5e-3 rel-L2, while interleaved-pair RoPE, the h % 3 head mapping, a missing
causal mask and theta 1e5 each miss it by more than 0.1; the decode rows reproduce the
full-sequence forward; zero-factor corrections are bitwise no-ops; the correction delta at
one projection is exact; the 4-bit trace equals F.linear(norm1, dequantize()); the tied
logits equal F.rms_norm + F.linear.
"""
import numpy as np
import torch
import torch.nn.functional as F

from oracle import lowbit_oracle as lo

PROJECTIONS = ('self_attn.q_proj.weight', 'self_attn.k_proj.weight', 'self_attn.v_proj.weight',
               'self_attn.o_proj.weight', 'mlp.gate_proj.weight', 'mlp.up_proj.weight', 'mlp.down_proj.weight')
HEADS, KV_HEADS, HEAD_DIM, HIDDEN = 9, 3, 64, 576


def rope_tables(theta, positions):
    """fp16 cos/sin [positions, 64] (rotate-half layout), as the reference builds them."""
    freq = 1.0 / (theta ** (torch.arange(0, HEAD_DIM, 2).float() / HEAD_DIM))
    ang = torch.outer(torch.arange(positions).float(), freq)
    ang = torch.cat((ang, ang), dim=-1)
    return ang.cos().half(), ang.sin().half()


class OracleLayer:
    """One decoder layer. weights: fp16 CPU tensors; packed: name -> (fmt, shape, group, data, scales);
    corrections: name -> (down fp16 [r,K], up fp16 [N,r]); protected: names kept in fp16."""

    def __init__(self, weights, packed=None, corrections=None, protected=(), *, theta=100000.0, capacity=64):
        self.w = {k: v.detach().float().half() for k, v in weights.items()}
        self.packed = packed or {}
        self.corr = corrections or {}
        self.protected = set(protected)
        self.cos, self.sin = rope_tables(theta, capacity)
        self.capacity = capacity
        self._weight_cache = {}

    def _weight(self, name):
        if name not in self._weight_cache:
            fmt, shape, group, data, scales = self.packed[name]
            if fmt == 'int8' and group == shape[1]:
                self._weight_cache[name] = ('f64', torch.from_numpy(lo.exact_weight(fmt, shape, group, data, scales)))
            else:
                self._weight_cache[name] = ('f32', torch.from_numpy(
                    lo.dequantize(fmt, shape, group, data, scales).astype(np.float32)))
        return self._weight_cache[name]

    def linear(self, v, name):
        if name in self.packed and name not in self.protected:
            kind, w = self._weight(name)
            out = (v.double() @ w.T).half() if kind == 'f64' else F.linear(v.float(), w).half()
            if name in self.corr:
                down, up = self.corr[name]
                z = F.linear(v.float(), down.float()).half()
                d = F.linear(z.float(), up.float()).half()
                out = (out + d).half()
            return out
        return F.linear(v.float(), self.w[name].float()).half()

    def norm(self, v, name):
        f = v.float()
        n = (f * torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)).half()
        return (n * self.w[name]).half()

    @staticmethod
    def _rotate(v, cos, sin):
        rot = torch.cat((-v[..., 32:], v[..., :32]), -1)
        return (v * cos + rot * sin).half()

    @staticmethod
    def _attend(q, k, v, mask):
        k = k.repeat_interleave(3, dim=1)
        v = v.repeat_interleave(3, dim=1)
        scores = (q.float() @ k.float().transpose(-1, -2)).half()
        scores = (scores * 0.125).half()
        probs = (scores + mask).float().softmax(-1).half()
        return (probs.float() @ v.float()).half()

    def _mlp(self, value, trace):
        n2 = self.norm(value, 'post_attention_layernorm.weight')
        trace['norm2'] = n2
        gate = self.linear(n2, 'mlp.gate_proj.weight')
        up = self.linear(n2, 'mlp.up_proj.weight')
        act = F.silu(gate.float()).half()
        hidden = (act * up).half()
        trace['gated'] = hidden
        delta = self.linear(hidden, 'mlp.down_proj.weight')
        trace['ffn_output'] = delta
        return (value + delta).half()

    def forward(self, x):
        """Full causal sequence x [B,S,576] fp16 -> (out, trace, keys [B,3,S,64], values)."""
        b, s, d = x.shape
        x = x.half()
        trace = {}
        n1 = self.norm(x, 'input_layernorm.weight')
        trace['norm1'] = n1
        q = self.linear(n1, 'self_attn.q_proj.weight').view(b, s, HEADS, HEAD_DIM).transpose(1, 2)
        k = self.linear(n1, 'self_attn.k_proj.weight').view(b, s, KV_HEADS, HEAD_DIM).transpose(1, 2)
        v = self.linear(n1, 'self_attn.v_proj.weight').view(b, s, KV_HEADS, HEAD_DIM).transpose(1, 2)
        cos, sin = self.cos[:s][None, None], self.sin[:s][None, None]
        q, k = self._rotate(q, cos, sin), self._rotate(k, cos, sin)
        trace['keys'], trace['values'] = k, v
        mask = torch.triu(torch.full((s, s), float('-inf')), diagonal=1)
        att = self._attend(q, k, v, mask).transpose(1, 2).reshape(b, s, d)
        trace['attention'] = att
        delta = self.linear(att, 'self_attn.o_proj.weight')
        trace['attention_output'] = delta
        value = (x + delta).half()
        trace['residual1'] = value
        out = self._mlp(value, trace)
        trace['output'] = out
        return out, trace, k, v

    def decode(self, x, keys, values, pos):
        """One token x [B,1,576] at position pos; keys/values [B,3,>=pos,64] hold 0..pos-1.
        Returns (out, keys', values') with the new row appended."""
        b = x.shape[0]
        x = x.half()
        trace = {}
        n1 = self.norm(x, 'input_layernorm.weight')
        q = self.linear(n1, 'self_attn.q_proj.weight').view(b, 1, HEADS, HEAD_DIM).transpose(1, 2)
        k = self.linear(n1, 'self_attn.k_proj.weight').view(b, 1, KV_HEADS, HEAD_DIM).transpose(1, 2)
        v = self.linear(n1, 'self_attn.v_proj.weight').view(b, 1, KV_HEADS, HEAD_DIM).transpose(1, 2)
        cos, sin = self.cos[pos:pos + 1][None, None], self.sin[pos:pos + 1][None, None]
        q, k = self._rotate(q, cos, sin), self._rotate(k, cos, sin)
        keys = torch.cat((keys[:, :, :pos], k), dim=2)
        values = torch.cat((values[:, :, :pos], v), dim=2)
        mask = torch.zeros(1, pos + 1)
        att = self._attend(q, keys, values, mask).transpose(1, 2).reshape(b, 1, HIDDEN)
        delta = self.linear(att, 'self_attn.o_proj.weight')
        value = (x + delta).half()
        return self._mlp(value, trace), keys, values


class OracleModel:
    """Stack + tied embedding / final norm endpoints, greedy generation with a KV cache.
    head: (fmt, shape, group, data, scales) of a quantized tied head, or None for the fp16 one;
    a quantized head is the projection linear above (W8 per-row exact q*s, 4-bit fp16(q*s))."""

    def __init__(self, layers, embedding, norm, head=None):
        self.layers = layers
        self.embedding = embedding.detach().float().half()
        self.norm_w = norm.detach().float().half()
        self.head = head

    def embed(self, ids):
        return F.embedding(ids, self.embedding)

    def logits(self, hidden):
        f = hidden.float()
        inv = torch.rsqrt(f.square().mean(-1, keepdim=True) + 1e-5)
        normalized = (f * inv).half() * self.norm_w
        if self.head is None:
            return F.linear(normalized, self.embedding)
        fmt, shape, group, data, scales = self.head
        if fmt == 'int8' and group == shape[1]:
            w = torch.from_numpy(lo.exact_weight(fmt, shape, group, data, scales))
            return (normalized.double() @ w.T).half()
        w = torch.from_numpy(lo.dequantize(fmt, shape, group, data, scales).astype(np.float32))
        return F.linear(normalized.float(), w).half()

    def prefill(self, ids):
        x = self.embed(ids)
        caches = []
        for layer in self.layers:
            x, _, k, v = layer.forward(x)
            caches.append((k, v))
        return x, caches

    def generate(self, ids, steps, forced=None):
        """Greedy: returns (tokens [steps], logits fp16 [steps, vocab]) for the steps after the prompt.
        forced: a token list to feed instead of the argmax (teacher forcing; logits as greedy)."""
        x, caches = self.prefill(ids)
        pos = ids.shape[1]
        logits = self.logits(x[:, -1:])[:, 0]
        tokens, all_logits = [], []
        for step in range(steps):
            tok = int(logits[0].float().argmax()) if forced is None else int(forced[step])
            tokens.append(tok)
            all_logits.append(logits[0].clone())
            if step == steps - 1:
                break
            h = self.embed(torch.tensor([[tok]]))
            new = []
            for layer, (k, v) in zip(self.layers, caches):
                h, k, v = layer.decode(h, k, v, pos)
                new.append((k, v))
            caches = new
            pos += 1
            logits = self.logits(h)[:, 0]
        return tokens, torch.stack(all_logits)
