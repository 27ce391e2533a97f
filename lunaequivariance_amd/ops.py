"""Dispatcher operators for ``torch.compile`` / export.

Mirror of the reference's ``lunatp::uvu_conv_forward`` / ``_backward``
custom ops (``src/lunatp/uvu_conv/interface.py:18-140``) and
``lunatp::uuu_conv_forward`` / ``_backward``
(``src/lunatp/uuu_conv/interface.py:15-150``) under the ``lunaeq_amd``
namespace: tensors, graph tables and a JSON string of the
static configuration go in; fake kernels give output shapes; autograd of the
forward op calls the backward op, and autograd of the backward op composes
forward and backward ops with cotangent-substituted arguments (the
convolution is multilinear), so compiled graphs differentiate to any order.
"""

from __future__ import annotations

import json
from dataclasses import dataclass
from functools import lru_cache

import torch

GRAPH_TABLES = ("src", "dst", "dst_rowptr", "src_rowptr", "edge_ids_by_src", "node_order", "source_node_order")


@dataclass
class GraphTables:
    """The subset of a LunaTPGraph the kernels read."""

    src: torch.Tensor
    dst: torch.Tensor
    dst_rowptr: torch.Tensor
    src_rowptr: torch.Tensor
    edge_ids_by_src: torch.Tensor
    node_order: torch.Tensor
    source_node_order: torch.Tensor
    num_nodes: int

    @property
    def num_edges(self) -> int:
        return int(self.src.numel())


def graph_tables(graph):
    return [getattr(graph, name) for name in GRAPH_TABLES]


def operator_config(op) -> str:
    """Static configuration of a prepared convolution as a graph constant."""
    meta = dict(op.meta)
    meta["generated_specs"] = [dict(s, terms=[list(t) for t in s["terms"]]) for s in meta["generated_specs"]]
    return json.dumps({"dtype": str(op.compute_dtype).split(".")[-1], "mode": op.mode, "meta": meta},
                      sort_keys=True)


@lru_cache(maxsize=128)
def restore_operator(config: str):
    from .uuu_conv import LunaTPUUUConv
    from .uvu_conv import LunaTPUVUConv

    data = json.loads(config)
    meta = data["meta"]
    meta["generated_specs"] = [dict(s, terms=[tuple(t) for t in s["terms"]]) for s in meta["generated_specs"]]
    cls = LunaTPUUUConv if data.get("mode") == "uuu_conv" else LunaTPUVUConv
    return cls(meta, dtype=getattr(torch, data["dtype"]))


@lru_cache(maxsize=128)
def _static(config: str):
    data = json.loads(config)
    from .uvu_conv import l0_feature_layout

    _, l0_dim = l0_feature_layout(data["meta"]["generated_specs"])
    return data["meta"]["out_dim"], l0_dim


def _tables(tables, num_nodes):
    return GraphTables(*tables, num_nodes=int(num_nodes))


def _register(prefix):
    """Forward and backward dispatcher ops ``lunaeq_amd::<prefix>_conv_*`` with autograd."""

    @torch.library.custom_op(f"lunaeq_amd::{prefix}_conv_forward", mutates_args=(),
                             schema="(Tensor x, Tensor y, Tensor w, Tensor? env, Tensor[] tables, SymInt num_nodes, "
                                    "bool return_l0, str config) -> (Tensor, Tensor?)")
    def conv_forward(x, y, w, env, tables, num_nodes, return_l0, config):
        out, l0 = restore_operator(config).launch_forward(x, y, w, _tables(tables, num_nodes), env, return_l0)
        return out, l0

    @conv_forward.register_fake
    def _conv_forward_fake(x, y, w, env, tables, num_nodes, return_l0, config):
        out_dim, l0_dim = _static(config)
        out = x.new_empty((num_nodes, out_dim))
        return out, (y.new_empty((y.shape[0], l0_dim)) if return_l0 else None)

    @torch.library.custom_op(f"lunaeq_amd::{prefix}_conv_backward", mutates_args=(),
                             schema="(Tensor x, Tensor y, Tensor w, Tensor? env, Tensor g, Tensor? gl0, Tensor[] tables, "
                                    "SymInt num_nodes, bool[] needs, str config) -> (Tensor?, Tensor?, Tensor?, Tensor?)")
    def conv_backward(x, y, w, env, g, gl0, tables, num_nodes, needs, config):
        return restore_operator(config).launch_backward(x, y, w, _tables(tables, num_nodes), g, env, gl0,
                                                        tuple(needs))

    @conv_backward.register_fake
    def _conv_backward_fake(x, y, w, env, g, gl0, tables, num_nodes, needs, config):
        return tuple(torch.empty_like(value) if need and value is not None else None
                     for value, need in zip((x, y, w, env), needs))

    def _forward_setup(ctx, inputs, output):
        x, y, w, env, tables, num_nodes, return_l0, config = inputs
        ctx.save_for_backward(x, y, w, env, *tables)
        ctx.num_nodes, ctx.config, ctx.return_l0 = num_nodes, config, return_l0
        ctx.table_count = len(tables)
        ctx.set_materialize_grads(False)

    def _forward_backward(ctx, g, gl0):
        x, y, w, env, *tables = ctx.saved_tensors
        if g is None:
            g = x.new_zeros((ctx.num_nodes, _static(ctx.config)[0]))
        needs = list(ctx.needs_input_grad[:4])
        gx, gy, gw, genv = conv_backward(x, y, w, env, g.contiguous(),
                                         None if gl0 is None else gl0.contiguous(),
                                         list(tables), ctx.num_nodes, needs, ctx.config)
        return gx, gy, gw, genv, [None] * ctx.table_count, None, None, None

    def _backward_setup(ctx, inputs, output):
        x, y, w, env, g, gl0, tables, num_nodes, needs, config = inputs
        ctx.save_for_backward(x, y, w, env, g, gl0, *tables)
        ctx.num_nodes, ctx.config = num_nodes, config
        ctx.table_count = len(tables)
        ctx.set_materialize_grads(False)

    def _backward_backward(ctx, rx, ry, rw, renv):
        x, y, w, env, g, gl0, *tables = ctx.saved_tensors
        need = ctx.needs_input_grad  # x, y, w, env, g, gl0, tables, num_nodes, needs, config
        want_l0 = gl0 is not None
        args = [x, y, w, env]
        dirs = [None if r is None else r.contiguous() for r in (rx, ry, rw)]
        dirs.append(None if (renv is None or env is None) else renv.contiguous())
        grads = [None] * 4
        hg = hl0 = None
        for slot, direction in enumerate(dirs):
            if direction is None:
                continue
            sub = list(args)
            sub[slot] = direction
            # Along a weight direction only the weighted paths vary.
            config = restore_operator(ctx.config).weight_linear().torch_config if slot == 2 else ctx.config
            scalar = want_l0 and slot != 3
            if need[4] or (need[5] and scalar):
                out, l0 = conv_forward(*sub, list(tables), ctx.num_nodes, scalar, config)
                hg = _add(hg, out)
                if scalar:
                    hl0 = _add(hl0, l0)
            wanted = [bool(need[o]) and o != slot and args[o] is not None for o in range(4)]
            if any(wanted):
                parts = conv_backward(*sub, g, gl0 if slot != 3 else None, list(tables), ctx.num_nodes, wanted,
                                      config)
                for o in range(4):
                    if wanted[o] and parts[o] is not None:
                        grads[o] = _add(grads[o], parts[o])
        return (*grads, hg if need[4] else None, hl0 if need[5] else None, [None] * ctx.table_count, None, None,
                None)

    conv_forward.register_autograd(_forward_backward, setup_context=_forward_setup)
    conv_backward.register_autograd(_backward_backward, setup_context=_backward_setup)
    return conv_forward, conv_backward


def _add(a, b):
    return b if a is None else (a if b is None else a + b)


conv_forward, conv_backward = _register("uvu")
uuu_conv_forward, uuu_conv_backward = _register("uuu")


__all__ = ["conv_forward", "conv_backward", "uuu_conv_forward", "uuu_conv_backward", "operator_config", "restore_operator", "graph_tables"]
