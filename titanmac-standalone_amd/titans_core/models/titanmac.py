"""TitanMAC language model (drop-in for models/titanmac.py).

Same constructor, submodules, parameters, buffers and state_dict keys as the reference
(models/titanmac.py:36-158), and the same forwards with the same outputs:

- ``forward`` dispatches to ``forward_mac`` / ``forward_mag`` / ``forward_mal`` when the neural
  memory is on (:554-600), and otherwise runs embeddings → [persistent | sequence] → blocks →
  norm → head (:601-686);
- ``forward_mac`` (:160-313) splits the sequence into segments. For each one it retrieves
  ``n_memory_tokens`` memory tokens from the segment mean, runs the blocks over
  [persistent | memory | segment], updates the memory (training or test-time memory) or only
  measures its loss, and gates the segment output by sigmoid(gate_proj(M*(y)));
- ``forward_mag`` (:315-432) and ``forward_mal`` (:434-547).

Every block op runs on the HIP kernels (RMSNorm, depthwise conv, tile-sparse attention,
Block-ELL MLP when configured), the neural memory's update on its HIP step, and the dense
projections and the LM head on hipBLASLt.

One change of schedule, not of result: when the memory is read-only (eval mode without
``enable_test_time_memory``), ``forward_mac``'s segments do not depend on each other. The
reference still runs them one after another, each as B sequences of S = Np + N_l + segment
tokens. Here all full segments run through the blocks as one batch of (n_segments·B)
sequences, and a shorter last segment as a second batch. That is the same arithmetic per
sequence, in a few large launches instead of many small ones. With updates on, segment i+1
reads the memory that segment i wrote, so they run in order as in the reference.
"""
from __future__ import annotations

from typing import Dict, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils.checkpoint import checkpoint

from ..blocks.norms import RMSNorm
from ..blocks.titan_block import TitanBlock
from ..config import TitanMACConfig
from ..memory.neural_memory import NeuralMemory


class TitanMAC(nn.Module):
    """Titan Memory-Augmented Context model: input_ids [B, T] → {"logits": [B, T, vocab], ...}."""

    def __init__(self, config: TitanMACConfig):
        super().__init__()
        self.config = config
        config.validate()
        if config.use_memory_bank:
            raise NotImplementedError(
                "use_memory_bank: the legacy MemoryBank is not part of this build (no forward of "
                "the reference reads it)")
        d = config.d_model
        self.embed_tokens = nn.Embedding(config.vocab_size, d)
        self.embed_positions = nn.Embedding(config.max_seq_len, d)
        if config.n_persistent > 0:
            self.persistent_tokens = nn.Parameter(torch.zeros(config.n_persistent, d))
        else:
            self.register_parameter("persistent_tokens", None)
        self.layers = nn.ModuleList([TitanBlock(config) for _ in range(config.n_layers)])
        self.norm = RMSNorm(d, eps=config.norm_eps)
        self.lm_head = nn.Linear(d, config.vocab_size, bias=False)
        if config.tie_weights:
            self.lm_head.weight = self.embed_tokens.weight
        self.memory_bank = None
        if config.use_neural_memory:
            d_mem = config.d_memory if config.d_memory is not None else d
            self.neural_memory = NeuralMemory(
                d_model=d, d_memory=d_mem, n_memory_layers=config.n_memory_layers,
                theta_lr=config.memory_theta_lr, forget_hidden=config.memory_forget_hidden,
                decay_hidden=config.memory_decay_hidden)
            self.memory_proj = nn.Linear(d_mem, d)
            self.gate_proj = nn.Linear(d_mem, d)
        else:
            self.neural_memory = None
            self.memory_proj = None
            self.gate_proj = None
        self.gradient_checkpointing = False
        self._block_graph = None
        self._init_weights()

    def _init_weights(self) -> None:
        """N(0, 0.02) embeddings, persistent tokens, untied head, memory projections (:140-158)."""
        nn.init.normal_(self.embed_tokens.weight, mean=0.0, std=0.02)
        nn.init.normal_(self.embed_positions.weight, mean=0.0, std=0.02)
        if self.persistent_tokens is not None:
            nn.init.normal_(self.persistent_tokens, mean=0.0, std=0.02)
        if not self.config.tie_weights:
            nn.init.normal_(self.lm_head.weight, mean=0.0, std=0.02)
        if self.memory_proj is not None:
            nn.init.normal_(self.memory_proj.weight, mean=0.0, std=0.02)
        if self.gate_proj is not None:
            nn.init.normal_(self.gate_proj.weight, mean=0.0, std=0.02)

    # ------------------------------------------------------------------ helpers

    def _embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        T = input_ids.shape[1]
        pos = torch.arange(T, device=input_ids.device)
        return self.embed_tokens(input_ids) + self.embed_positions(pos).unsqueeze(0)

    def _persistent(self, B: int) -> Optional[torch.Tensor]:
        if self.persistent_tokens is not None and self.config.n_persistent > 0:
            return self.persistent_tokens.unsqueeze(0).expand(B, -1, -1)
        return None

    def _blocks(self, y: torch.Tensor, layers=None) -> torch.Tensor:
        for layer in (self.layers if layers is None else layers):
            if self.gradient_checkpointing and self.training:
                y = checkpoint(lambda h, m=layer: m(h, attn_mask=None), y, use_reentrant=False)
            else:
                y = layer(y, attn_mask=None)
        return y

    # ------------------------------------------------------------------ block-stack graph

    def _tensor_ptrs(self):
        return tuple(t.data_ptr() for t in list(self.parameters()) + list(self.buffers()))

    def capture_block_graph(self, batch: int, seq_len: Optional[int] = None) -> None:
        """Capture the layer stack for one input shape [batch, seq_len, d_model] in a HIP graph.

        For eval forwards with test-time memory, whose segments run the layers one after
        another with small batches: there the host's launch rate, not the GPU, sets the pace,
        and one graph replay replaces a few hundred launches. seq_len defaults to the MAC
        segment shape, n_persistent + n_memory_tokens + segment_size. Without gradients and
        outside training, ``forward_mac`` then replays the graph for every input of that
        shape, dtype and device; other inputs, and any call after a parameter or buffer was
        replaced (not updated in place, e.g. by ``.to()``), run the layers eagerly again.
        Results are bit-identical to the eager layers (the same kernels on the same data).
        Capture again after such changes; ``release_block_graph`` frees the graph.
        """
        if seq_len is None:
            seq_len = self.config.n_persistent + self.config.n_memory_tokens + self.config.segment_size
        p = next(self.parameters())
        if not p.is_cuda:
            raise RuntimeError("capture_block_graph needs the model on a GPU")
        self.release_block_graph()
        static_in = torch.zeros(batch, seq_len, self.config.d_model, dtype=p.dtype, device=p.device)
        was_training = self.training
        self.eval()
        try:
            side = torch.cuda.Stream(device=p.device)
            side.wait_stream(torch.cuda.current_stream(p.device))
            with torch.cuda.stream(side), torch.no_grad():
                for _ in range(2):  # warm-up outside the capture (lazy caches, libraries)
                    self._blocks(static_in)
            torch.cuda.current_stream(p.device).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph), torch.no_grad():
                static_out = self._blocks(static_in)
        finally:
            self.train(was_training)
        self._block_graph = {"graph": graph, "in": static_in, "out": static_out,
                             "ptrs": self._tensor_ptrs(), "replays": 0}

    def release_block_graph(self) -> None:
        self._block_graph = None

    def _graph_blocks(self, parts) -> torch.Tensor:
        """blocks(cat(parts, dim=1)) through the captured graph when it applies; the result
        stays valid until the next call (the graph's output buffer)."""
        gr = self._block_graph
        if gr is not None and not self.training and not torch.is_grad_enabled():
            st = gr["in"]
            if (all(t.dtype == st.dtype and t.device == st.device for t in parts)
                    and sum(t.shape[1] for t in parts) == st.shape[1]
                    and all(t.shape[0] == st.shape[0] and t.shape[2] == st.shape[2] for t in parts)
                    and self._tensor_ptrs() == gr["ptrs"]):
                torch.cat(parts, dim=1, out=st)
                gr["graph"].replay()
                gr["replays"] += 1
                return gr["out"]
        return self._blocks(torch.cat(parts, dim=1))

    def _memory_step(self, y: torch.Tensor) -> torch.Tensor:
        if self.training or self.config.enable_test_time_memory:
            return self.neural_memory.update(y)
        return self.neural_memory.compute_loss(y)

    def _output(self, logits: torch.Tensor, labels: Optional[torch.Tensor],
                memory_loss: Optional[torch.Tensor]) -> Dict[str, torch.Tensor]:
        out = {"logits": logits}
        if memory_loss is not None:
            out["memory_loss"] = memory_loss
        if labels is not None:
            ce = F.cross_entropy(logits[..., :-1, :].contiguous().reshape(-1, self.config.vocab_size),
                                 labels[..., 1:].contiguous().reshape(-1), reduction="mean",
                                 ignore_index=-100)
            if memory_loss is None:
                out["loss"] = ce
            else:
                out["ce_loss"] = ce
                out["loss"] = ce + memory_loss
        return out

    # ------------------------------------------------------------------ MAC

    def _mac_segments(self, xs: torch.Tensor, persistent_row: Optional[torch.Tensor],
                      n_seq: int, acc: torch.Tensor) -> torch.Tensor:
        """Blocks and gated output for a batch of independent segments xs [n·B, L, d]
        (segment-major) against a read-only memory; adds each segment's memory loss
        F.mse_loss(M(W_K y), W_V y) over its B sequences to ``acc`` in order, as the reference's
        per-segment loop does. Returns o [n·B, L, d]."""
        nl = self.config.n_memory_tokens
        NB, L, d = xs.shape
        h = self.memory_proj(self.neural_memory.retrieve(xs.mean(dim=1, keepdim=True)))
        parts = [h.expand(NB, nl, d), xs]
        if persistent_row is not None:
            parts.insert(0, persistent_row.unsqueeze(0).expand(NB, -1, -1))
        y = self._blocks(torch.cat(parts, dim=1))
        ys = y[:, y.shape[1] - L:]
        nm = self.neural_memory
        pred, target = nm.memory_mlp(nm.W_K(ys)), nm.W_V(ys)
        B = NB // n_seq
        for s in range(n_seq):
            acc.add_(F.mse_loss(pred[s * B:(s + 1) * B], target[s * B:(s + 1) * B]))
        gate = torch.sigmoid(self.gate_proj(nm.retrieve(ys)))
        return ys * gate

    def forward_mac(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                    attention_mask: Optional[torch.Tensor] = None) -> Dict[str, torch.Tensor]:
        """Memory as Context (models/titanmac.py:160-313)."""
        if self.neural_memory is None:
            raise ValueError("forward_mac requires use_neural_memory=True")
        B, T = input_ids.shape
        x = self._embed(input_ids)
        seg = self.config.segment_size
        nl = self.config.n_memory_tokens
        n_segments = (T + seg - 1) // seg
        persistent = self._persistent(B)
        Np = 0 if persistent is None else self.config.n_persistent

        if not (self.training or self.config.enable_test_time_memory):
            # Read-only memory: all full segments in one batch, the remainder in another.
            n_full, tail = divmod(T, seg)
            prow = None if persistent is None else self.persistent_tokens
            outs, acc = [], torch.zeros(1, device=x.device, dtype=x.dtype)
            if n_full:
                xs = x[:, :n_full * seg].reshape(B, n_full, seg, -1).transpose(0, 1)
                o = self._mac_segments(xs.reshape(n_full * B, seg, -1), prow, n_full, acc)
                outs.append(o.reshape(n_full, B, seg, -1).transpose(0, 1).reshape(B, n_full * seg, -1))
            if tail:
                outs.append(self._mac_segments(x[:, n_full * seg:], prow, 1, acc))
            o = x if not outs else (outs[0] if len(outs) == 1 else torch.cat(outs, dim=1))
            memory_loss = (acc / n_segments).squeeze()  # nan for T = 0, as in the reference
        else:
            o = torch.empty_like(x)
            acc = torch.zeros(1, device=x.device, dtype=x.dtype)
            for s in range(n_segments):
                a, b = s * seg, min(s * seg + seg, T)
                xs = x[:, a:b]
                q = xs.mean(dim=1, keepdim=True).expand(B, nl, -1)
                h = self.memory_proj(self.neural_memory.retrieve(q))
                parts = [h, xs] if persistent is None else [persistent, h, xs]
                y = self._graph_blocks(parts)
                ys = y[:, Np + nl:]
                acc = acc + self._memory_step(ys)
                gate = torch.sigmoid(self.gate_proj(self.neural_memory.retrieve(ys)))
                o[:, a:b] = ys * gate
            memory_loss = (acc / n_segments).squeeze()
        logits = self.lm_head(self.norm(o))
        return self._output(logits, labels, memory_loss)

    # ------------------------------------------------------------------ MAG / MAL

    def forward_mag(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                    attention_mask: Optional[torch.Tensor] = None) -> Dict[str, torch.Tensor]:
        """Memory as Gate (models/titanmac.py:315-432): o = blocks(x̃) ⊙ sigmoid(gate_proj(M*(x̃)))."""
        if self.neural_memory is None:
            raise ValueError("forward_mag requires use_neural_memory=True")
        B = input_ids.shape[0]
        x = self._embed(input_ids)
        persistent = self._persistent(B)
        xc = x if persistent is None else torch.cat([persistent, x], dim=1)
        gate = torch.sigmoid(self.gate_proj(self.neural_memory.retrieve(xc)))
        y = self._blocks(xc)
        o = y * gate
        Np = 0 if persistent is None else self.config.n_persistent
        memory_loss = self._memory_step(y[:, Np:])
        logits = self.lm_head(self.norm(o)[:, Np:])
        return self._output(logits, labels, memory_loss)

    def forward_mal(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                    attention_mask: Optional[torch.Tensor] = None) -> Dict[str, torch.Tensor]:
        """Memory as Layer (models/titanmac.py:434-547): even layers are blocks, odd layers add
        memory_proj(M*(y))."""
        if self.neural_memory is None:
            raise ValueError("forward_mal requires use_neural_memory=True")
        B = input_ids.shape[0]
        x = self._embed(input_ids)
        persistent = self._persistent(B)
        y = x if persistent is None else torch.cat([persistent, x], dim=1)
        for i, layer in enumerate(self.layers):
            if i % 2 == 0:
                y = self._blocks(y, [layer])
            else:
                y = y + self.memory_proj(self.neural_memory.retrieve(y))
        Np = 0 if persistent is None else self.config.n_persistent
        memory_loss = self._memory_step(y[:, Np:])
        logits = self.lm_head(self.norm(y)[:, Np:])
        return self._output(logits, labels, memory_loss)

    def forward_with_memory(self, *args, **kwargs):
        """Alias of forward_mac (models/titanmac.py:550-552)."""
        return self.forward_mac(*args, **kwargs)

    # ------------------------------------------------------------------ dispatch

    def forward(self, input_ids: torch.Tensor, labels: Optional[torch.Tensor] = None,
                attention_mask: Optional[torch.Tensor] = None) -> Dict[str, torch.Tensor]:
        if self.neural_memory is not None and self.config.use_neural_memory:
            variant = self.config.titans_variant
            if variant == "MAC":
                return self.forward_mac(input_ids, labels, attention_mask)
            if variant == "MAG":
                return self.forward_mag(input_ids, labels, attention_mask)
            if variant == "MAL":
                return self.forward_mal(input_ids, labels, attention_mask)
            raise ValueError(f"Unknown titans_variant: {variant}")
        B = input_ids.shape[0]
        x = self._embed(input_ids)
        persistent = self._persistent(B)
        if persistent is not None:
            x = torch.cat([persistent, x], dim=1)
        logits = self.lm_head(self.norm(self._blocks(x)))
        if persistent is not None:
            logits = logits[:, self.config.n_persistent:, :]
        return self._output(logits, labels, None)

    # ------------------------------------------------------------------ utilities

    def _should_update_memory(self) -> bool:
        return True if self.training else self.config.enable_test_time_memory

    def get_num_params(self, non_embedding: bool = True) -> int:
        """Parameter count, optionally without the embeddings (and an untied head) (:701-730)."""
        total = sum(p.numel() for p in self.parameters())
        if not non_embedding:
            return total
        emb = self.embed_tokens.weight.numel() + self.embed_positions.weight.numel()
        if not self.config.tie_weights:
            emb += self.lm_head.weight.numel()
        return total - emb

    def reset_memory(self) -> None:
        """Resets the MemoryBank in the reference; there is none here (see __init__)."""

    def get_memory_stats(self) -> Optional[Dict[str, float]]:
        return None

    def enable_gradient_checkpointing(self) -> None:
        self.gradient_checkpointing = True

    def disable_gradient_checkpointing(self) -> None:
        self.gradient_checkpointing = False
