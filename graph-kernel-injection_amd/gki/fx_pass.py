"""torch.fx pass that swaps scaled-dot-product attention for the gfx950 op.

Behavioural mirror of the reference pass (``fx_compiler_pass.py:49-653``):

* ``StandardAttention`` / ``SingleLayerTransformer`` -- the eager input modules.
* ``_InjectedTritonAttention`` -- the installed child module (name kept for
  drop-in compatibility); its ``forward`` calls :func:`block_sparse_attention`,
  which now launches the HIP kernels. Its ``block_mask`` buffer is
  non-persistent and follows ``.to(device)``.
* ``BlockSparseAttentionInjector(InjectionConfig).transform(model)`` traces the
  model and rewrites (a) the eager motif
  ``matmul(q, k.transpose) -> [mul|truediv by a static scalar] -> softmax(-1)
  -> matmul(., v)`` and (b) ``F.scaled_dot_product_attention(..., is_causal=True)``
  without dropout and with a static scale into ``call_module`` nodes named
  ``_triton_attn_{i}`` (eager matches numbered first). No match raises
  ``RuntimeError("No scaled-dot-product-attention subgraph found ...")``.
"""

from __future__ import annotations

import math
import operator
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.fx as fx
import torch.nn as nn
import torch.nn.functional as F  # noqa: N812

from .masks import StreamingMaskSpec, make_streaming_mask
from .ops import block_sparse_attention


# ---------------------------------------------------------------------------
# Input modules (fx_compiler_pass.py:54-116)
# ---------------------------------------------------------------------------


class StandardAttention(nn.Module):
    """Textbook ``softmax(Q K^T / sqrt(d)) V`` written in eager PyTorch."""

    def __init__(self, head_dim: int) -> None:
        super().__init__()
        if head_dim <= 0:
            raise ValueError("head_dim must be positive")
        self.head_dim = head_dim
        # a plain Python float, so tracing folds it into the graph as a constant
        self.inv_sqrt_d = 1.0 / math.sqrt(head_dim)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        scores = torch.matmul(q, k.transpose(-2, -1)) * self.inv_sqrt_d
        probs = torch.softmax(scores, dim=-1)
        return torch.matmul(probs, v)


class SingleLayerTransformer(nn.Module):
    """q/k/v/out projections around :class:`StandardAttention`."""

    def __init__(self, head_dim: int, model_dim: int) -> None:
        super().__init__()
        self.q_proj = nn.Linear(model_dim, model_dim, bias=False)
        self.k_proj = nn.Linear(model_dim, model_dim, bias=False)
        self.v_proj = nn.Linear(model_dim, model_dim, bias=False)
        self.out_proj = nn.Linear(model_dim, model_dim, bias=False)
        self.attn = StandardAttention(head_dim)
        self.num_heads = model_dim // head_dim
        self.head_dim = head_dim

    def _split(self, x: torch.Tensor) -> torch.Tensor:
        B, N, _ = x.shape
        return x.view(B, N, self.num_heads, self.head_dim).transpose(1, 2)

    def _merge(self, x: torch.Tensor) -> torch.Tensor:
        return x.transpose(1, 2).contiguous().flatten(-2)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        q = self._split(self.q_proj(x))
        k = self._split(self.k_proj(x))
        v = self._split(self.v_proj(x))
        return self.out_proj(self._merge(self.attn(q, k, v)))


# ---------------------------------------------------------------------------
# Installed module (fx_compiler_pass.py:124-163)
# ---------------------------------------------------------------------------


class _InjectedTritonAttention(nn.Module):
    """Child module the pass installs; forwards to the gfx950 op."""

    def __init__(
        self,
        block_mask: torch.Tensor,
        softmax_scale: float,
        block_m: int,
        block_n: int,
        is_causal: bool = False,
        sink_size: int = 0,
        window_size: int = 0,
        enable_gqa: bool = False,
    ) -> None:
        super().__init__()
        self.register_buffer("block_mask", block_mask, persistent=False)
        self.softmax_scale = float(softmax_scale)
        self.block_m = int(block_m)
        self.block_n = int(block_n)
        self.is_causal = bool(is_causal)
        self.sink_size = int(sink_size)
        self.window_size = int(window_size)
        # grouped-query K/V (fewer heads than Q), as SDPA's enable_gqa; not in the
        # reference module, whose op requires equal head counts
        self.enable_gqa = bool(enable_gqa)

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return block_sparse_attention(
            q, k, v, self.block_mask,
            softmax_scale=self.softmax_scale,
            block_m=self.block_m,
            block_n=self.block_n,
            is_causal=self.is_causal,
            sink_size=self.sink_size,
            window_size=self.window_size,
            enable_gqa=self.enable_gqa,
        )


# ---------------------------------------------------------------------------
# The pass (fx_compiler_pass.py:171-621)
# ---------------------------------------------------------------------------


@dataclass
class InjectionConfig:
    """Configuration of :class:`BlockSparseAttentionInjector`.

    ``custom_mask`` (a pre-built block mask) takes precedence over
    ``streaming``; one of them is required. ``head_dim`` only sets the default
    SDPA scale ``1/sqrt(head_dim)``. The mask is always built on the CPU and
    follows the rewritten module's ``.to(device)``.
    """

    seq_len_q: int
    seq_len_kv: int
    head_dim: int
    streaming: Optional[StreamingMaskSpec] = None
    custom_mask: Optional[torch.Tensor] = None
    block_m: int = 64
    block_n: int = 64
    device: str | torch.device = "cuda"


@dataclass
class _AttentionMatch:
    q_node: fx.Node
    k_node: fx.Node
    v_node: fx.Node
    transpose_node: fx.Node
    qk_node: fx.Node
    scale_node: Optional[fx.Node]
    softmax_node: fx.Node
    pv_node: fx.Node
    scale_value: float


@dataclass
class _SDPAMatch:
    sdpa_node: fx.Node
    q_node: fx.Node
    k_node: fx.Node
    v_node: fx.Node
    is_causal: bool
    scale_value: Optional[float]
    enable_gqa: bool = False


_MATMULS = (torch.matmul, operator.matmul)
_SCALES = (operator.mul, torch.mul, operator.truediv, torch.div)
_DIVIDES = (operator.truediv, torch.div)
_SOFTMAX_FNS = (torch.softmax, F.softmax)


def _calls(node: fx.Node, targets) -> bool:
    return node.op == "call_function" and node.target in targets


def _is_softmax(node: fx.Node) -> bool:
    return _calls(node, _SOFTMAX_FNS) or (node.op == "call_method" and node.target == "softmax")


def _is_transpose(node: fx.Node) -> bool:
    if node.op == "call_method":
        return node.target in ("transpose", "mT")
    return node.op == "call_function" and node.target is torch.transpose


def _is_sdpa(node: fx.Node) -> bool:
    return node.op == "call_function" and node.target is F.scaled_dot_product_attention


def _arg(node: fx.Node, name: str, position: int, default: object) -> object:
    """SDPA argument by keyword or position:
    (query, key, value, attn_mask, dropout_p, is_causal, scale, enable_gqa)."""
    if name in node.kwargs:
        return node.kwargs[name]
    return node.args[position] if len(node.args) > position else default


def _literal_scale(node: fx.Node) -> Optional[float]:
    """First numeric literal among the scale node's args, scanning left to right;
    ``None`` if a ``get_attr`` comes first or there is no literal."""
    for a in node.args:
        if isinstance(a, (int, float)):
            return float(a)
        if isinstance(a, fx.Node) and a.op == "get_attr":
            return None
    return None


def _safe_erase(graph: fx.Graph, node: fx.Node) -> None:
    """Erase ``node`` only when nothing uses it any more."""
    if not node.users:
        graph.erase_node(node)


class BlockSparseAttentionInjector:
    """Rewrites attention subgraphs of a module into the gfx950 op."""

    def __init__(self, config: InjectionConfig) -> None:
        self.cfg = config
        self._mask = self._build_mask()

    def _build_mask(self) -> torch.Tensor:
        """CPU int32 block mask: ``custom_mask`` if given, else StreamingLLM."""
        if self.cfg.custom_mask is not None:
            return self.cfg.custom_mask.detach().to(device="cpu", dtype=torch.int32).contiguous()
        if self.cfg.streaming is None:
            raise ValueError("Must supply either `streaming` or `custom_mask`")
        return make_streaming_mask(
            self.cfg.seq_len_q, self.cfg.seq_len_kv, self.cfg.streaming,
            self.cfg.block_m, self.cfg.block_n, device="cpu",
        )

    # -- matching ------------------------------------------------------------

    @staticmethod
    def _resolve_scalar(scale_node: fx.Node, owner: fx.GraphModule) -> Optional[float]:
        """Value of a ``get_attr`` scale operand: a number or a 1-element tensor."""
        for a in scale_node.args:
            if isinstance(a, fx.Node) and a.op == "get_attr":
                value = getattr(owner, a.target, None)
                if isinstance(value, (int, float)):
                    return float(value)
                if isinstance(value, torch.Tensor) and value.numel() == 1:
                    return float(value.item())
        return None

    @staticmethod
    def _match_attention_subgraph(graph: fx.Graph, owner: fx.GraphModule) -> List[_AttentionMatch]:
        found: List[_AttentionMatch] = []
        for sm in graph.nodes:
            if not _is_softmax(sm):
                continue
            dim = sm.kwargs.get("dim")
            if dim is None and len(sm.args) >= 2:
                dim = sm.args[1]
            if dim is not None and dim != -1:
                continue
            src = sm.args[0] if sm.args else None
            if not isinstance(src, fx.Node):
                continue
            scale_node: Optional[fx.Node] = None
            scale = 1.0
            qk = src
            if _calls(src, _SCALES):
                scale_node = src
                qk = src.args[0]
                value = _literal_scale(src)
                if value is None:
                    value = BlockSparseAttentionInjector._resolve_scalar(src, owner)
                if value is None:
                    continue
                scale = 1.0 / value if src.target in _DIVIDES else value
            if not (isinstance(qk, fx.Node) and _calls(qk, _MATMULS)):
                continue
            q, kt = qk.args[0], qk.args[1]
            if not (isinstance(q, fx.Node) and isinstance(kt, fx.Node) and _is_transpose(kt)):
                continue
            k = kt.args[0]
            if not isinstance(k, fx.Node):
                continue
            consumers = list(sm.users)
            if len(consumers) != 1:
                continue
            pv = consumers[0]
            if not _calls(pv, _MATMULS) or pv.args[0] is not sm:
                continue
            v = pv.args[1]
            if not isinstance(v, fx.Node):
                continue
            found.append(_AttentionMatch(q, k, v, kt, qk, scale_node, sm, pv, scale))
        return found

    @staticmethod
    def _match_sdpa_subgraph(graph: fx.Graph) -> List[_SDPAMatch]:
        found: List[_SDPAMatch] = []
        for node in graph.nodes:
            if not _is_sdpa(node) or len(node.args) < 3:
                continue
            q, k, v = node.args[:3]
            if not all(isinstance(x, fx.Node) for x in (q, k, v)):
                continue
            if not bool(_arg(node, "is_causal", 5, False)):
                continue  # a non-causal SDPA may carry a dynamic mask: refuse
            dropout = _arg(node, "dropout_p", 4, 0.0)
            if isinstance(dropout, (int, float)) and float(dropout) != 0.0:
                continue
            scale = _arg(node, "scale", 6, None)
            if scale is not None and not isinstance(scale, (int, float)):
                continue  # dynamic scale
            gqa = _arg(node, "enable_gqa", 7, False)
            if not isinstance(gqa, bool):
                continue  # dynamic enable_gqa
            found.append(_SDPAMatch(node, q, k, v, True, None if scale is None else float(scale),
                                    gqa))
        return found

    # -- rewriting -----------------------------------------------------------

    def _streaming_params(self, default_window: int) -> tuple:
        s = self.cfg.streaming
        return (s.sink_size, s.window_size) if s is not None else (0, default_window)

    def _install(self, gm: fx.GraphModule, index: int, anchor: fx.Node, qkv: tuple,
                 scale: float, is_causal: bool, sink: int, window: int,
                 enable_gqa: bool = False) -> fx.Node:
        name = f"_triton_attn_{index}"
        gm.add_submodule(name, _InjectedTritonAttention(
            block_mask=self._mask, softmax_scale=scale,
            block_m=self.cfg.block_m, block_n=self.cfg.block_n,
            is_causal=is_causal, sink_size=sink, window_size=window, enable_gqa=enable_gqa,
        ))
        with gm.graph.inserting_before(anchor):
            new = gm.graph.call_module(name, args=qkv)
        anchor.replace_all_uses_with(new)
        return new

    def _install_sdpa_match(self, gm: fx.GraphModule, match: _SDPAMatch, index: int) -> None:
        scale = match.scale_value
        if scale is None:
            scale = 1.0 / math.sqrt(self.cfg.head_dim)
        # causal SDPA without StreamingLLM config = plain causal: window spans all keys
        sink, window = self._streaming_params(self.cfg.seq_len_kv)
        self._install(gm, index, match.sdpa_node, (match.q_node, match.k_node, match.v_node),
                      scale, match.is_causal, sink, window, match.enable_gqa)
        _safe_erase(gm.graph, match.sdpa_node)

    def _install_match(self, gm: fx.GraphModule, match: _AttentionMatch, index: int) -> None:
        streaming = self.cfg.streaming is not None
        sink, window = self._streaming_params(0)
        self._install(gm, index, match.pv_node, (match.q_node, match.k_node, match.v_node),
                      match.scale_value, streaming, sink, window)
        for node in (match.pv_node, match.softmax_node, match.scale_node, match.qk_node,
                     match.transpose_node):
            if node is not None:
                _safe_erase(gm.graph, node)

    def transform(self, model: nn.Module) -> fx.GraphModule:
        """Trace ``model`` and return a rewritten ``fx.GraphModule`` (input untouched)."""
        traced = fx.symbolic_trace(model)
        eager = self._match_attention_subgraph(traced.graph, traced)
        sdpa = self._match_sdpa_subgraph(traced.graph)
        if not eager and not sdpa:
            raise RuntimeError(
                "No scaled-dot-product-attention subgraph found "
                "(neither the eager softmax(QKᵀ·s)V motif nor an "
                "F.scaled_dot_product_attention(is_causal=True) call)."
            )
        # indices: eager matches 0..E-1, SDPA matches E..; rewrite last-to-first so
        # a later match still sees its producers' original nodes
        for offset, match in reversed(list(enumerate(sdpa))):
            self._install_sdpa_match(traced, match, index=len(eager) + offset)
        for idx, match in reversed(list(enumerate(eager))):
            self._install_match(traced, match, index=idx)
        traced.graph.lint()
        traced.recompile()
        return traced


def pretty_print_graph(gm: fx.GraphModule, header: str = "") -> str:
    """Generated source of ``gm`` plus a tally of node kinds."""
    lines: List[str] = [f"=== {header} ==="] if header else []
    lines.append(gm.graph.python_code(root_module="self").src.strip())
    tally: dict = {}
    for node in gm.graph.nodes:
        tally[node.op] = tally.get(node.op, 0) + 1
    lines.append("# node tally: " + ", ".join(f"{k}={v}" for k, v in sorted(tally.items())))
    return "\n".join(lines)
