"""HIP-graph decode harness for the attention path, mirroring
ModelRunner.capture_cudagraph / run_model (nanovllm/engine/model_runner.py:260-336).

The reference captures the whole model's decode step once per batch size in
graph_bs = [1, 2, 4, 8] + [16, 32, ..., max_bs] (model_runner.py:305), all graphs
sharing one memory pool, over static buffers sized for max_bs and
ceil(max_model_len / block_size) table columns (:296-304).  run_model picks the
smallest captured size >= bs, zeroes the static buffers, copies the live rows in
and replays (:266-281).  Batches above max_bs (or 512) run eagerly.

Here the captured step is the attention path of L decoder layers: for each
layer, Attention.forward(q, k, v) under the decode Context, i.e. store_kvcache of
the new token then paged decode (attention.py:58-79).  q/k/v of the step are
static inputs (in the model they come from the layer's projection).

Padding of the slot mapping (reference quirk Q1).  The reference zero-fills it,
so padded rows write their K/V into slot 0, which may belong to a live sequence.
pad_slot=0 reproduces that exactly: each layer runs the reference's two calls
(store, then decode), so a live sequence owning slot 0 reads the padded row as
the reference's does.  The default pad_slot=-1 is skipped by the store: padded
rows leave the cache alone and produce zero rows, and with no padded row writing
a slot, each layer's store runs inside its decode launch (Attention's
fuse_decode_store), one graph node fewer per layer.
"""
from __future__ import annotations

import torch

from ..layers.attention import Attention
from ..utils.context import reset_context, set_context


def graph_batch_sizes(max_bs: int) -> list[int]:
    """The captured batch sizes of model_runner.py:305."""
    return [x for x in [1, 2, 4, 8] if x <= max_bs] + list(range(16, max_bs + 1, 16))


def pick_graph_size(graph_bs: list[int], bs: int) -> int | None:
    """Smallest captured size that fits bs (model_runner.py:269), None if none does."""
    return next((x for x in graph_bs if x >= bs), None)


class DecodeGraphs:
    """Captured decode steps of `layers` (Attention modules whose k_cache/v_cache are
    already bound), replayed by run()."""

    def __init__(self, layers: list[Attention], max_bs: int, max_num_blocks: int, device=None,
                 pad_slot: int = -1):
        if not layers:
            raise ValueError("at least one Attention layer")
        self.layers = layers
        self.max_bs = min(max_bs, 512)
        self.max_num_blocks = max_num_blocks
        self.pad_slot = pad_slot
        a = layers[0]
        dev = device or a.k_cache.device
        nh, nkv, d = a.num_heads, a.num_kv_heads, a.head_dim
        mb = self.max_bs
        self.q = torch.zeros(mb, nh * d, dtype=torch.bfloat16, device=dev)
        self.k = torch.zeros(mb, nkv * d, dtype=torch.bfloat16, device=dev)
        self.v = torch.zeros(mb, nkv * d, dtype=torch.bfloat16, device=dev)
        self.slot_mapping = torch.full((mb,), pad_slot, dtype=torch.int32, device=dev)
        self.context_lens = torch.zeros(mb, dtype=torch.int32, device=dev)
        self.block_tables = torch.zeros(mb, max_num_blocks, dtype=torch.int32, device=dev)
        # per graph size: the layers' outputs as the captured step produced them
        # (graph-pool memory, rewritten by every replay of that graph)
        self.layer_outputs: dict[int, list[torch.Tensor]] = {}
        self.graph_bs = graph_batch_sizes(self.max_bs)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.pool = None

    def _call_layers(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> list[torch.Tensor]:
        """Every layer's forward, fused store+decode only under -1 padding."""
        outs = []
        for layer in self.layers:
            prev = layer.fuse_decode_store
            layer.fuse_decode_store = self.pad_slot < 0
            try:
                outs.append(layer(q, k, v))
            finally:
                layer.fuse_decode_store = prev
        return outs

    def _step(self, bs: int) -> list[torch.Tensor]:
        return self._call_layers(self.q[:bs], self.k[:bs], self.v[:bs])

    @torch.inference_mode()
    def capture(self) -> "DecodeGraphs":
        """Capture one graph per size, largest first, sharing one pool (model_runner.py:307-322)."""
        for bs in reversed(self.graph_bs):
            g = torch.cuda.CUDAGraph()
            set_context(False, slot_mapping=self.slot_mapping[:bs], context_lens=self.context_lens[:bs],
                        block_tables=self.block_tables[:bs])
            self._step(bs)  # warmup
            with torch.cuda.graph(g, self.pool):
                self.layer_outputs[bs] = self._step(bs)
            if self.pool is None:
                self.pool = g.pool()
            self.graphs[bs] = g
            torch.cuda.synchronize()
            reset_context()
        return self

    @torch.inference_mode()
    def run(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
            context_lens: torch.Tensor, block_tables: torch.Tensor) -> list[torch.Tensor]:
        """One decode step of every layer for bs = q.shape[0] rows; returns the L layers'
        (bs, nh*d) outputs.  From a graph these are views of the graph's own output tensors,
        valid until its next replay (as run_model returns graph_vars["outputs"][:bs],
        model_runner.py:281).  Sizes above the largest graph run eagerly
        (model_runner.py:264-265)."""
        bs = q.shape[0]
        size = pick_graph_size(self.graph_bs, bs)
        if size is None or block_tables.shape[1] > self.max_num_blocks:
            set_context(False, slot_mapping=slot_mapping, context_lens=context_lens, block_tables=block_tables)
            try:
                return self._call_layers(q, k, v)
            finally:
                reset_context()
        # static buffers: zero, live rows in (model_runner.py:271-280); slots padded with pad_slot
        self.q.zero_()
        self.k.zero_()
        self.v.zero_()
        self.slot_mapping.fill_(self.pad_slot)
        self.context_lens.zero_()
        self.block_tables.zero_()
        self.q[:bs] = q.reshape(bs, -1)
        self.k[:bs] = k.reshape(bs, -1)
        self.v[:bs] = v.reshape(bs, -1)
        self.slot_mapping[:bs] = slot_mapping
        self.context_lens[:bs] = context_lens
        self.block_tables[:bs, : block_tables.shape[1]] = block_tables
        self.graphs[size].replay()
        return [o[:bs] for o in self.layer_outputs[size]]
