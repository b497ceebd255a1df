"""IR producer: a ``torch.export`` graph written out in the reference's IR schema.

The reference gets its IR from ``torch_ir.extract_ir`` (third-party ``pytorch-ir``
0.2.2, absent here), called as ``extract_ir(wrapper, example_inputs,
model_name=...)`` (`examples/extract_qwen_ir.py:222,255`). ``extract_ir`` here
has the same signature and writes the schema the rest of the path reads
(`npu_compiler/ir_reader.py:46-94`): ``graph_inputs`` / ``graph_outputs`` /
``weights`` / ``weight_name_mapping`` / ``nodes`` / ``constants``.

How an exported node becomes an IR node (the convention
``npu_runtime.aten_executor.bind_arguments`` reads back):

* ``op_type`` is the overload's name, ``aten.<op>.<overload>``;
* schema arguments of type ``Tensor`` / ``Tensor[]`` that hold graph values go to
  ``inputs`` in schema order; a Python scalar passed for a ``Tensor`` argument
  (``add.Tensor(x, 1e-6)``) and an absent optional tensor go to ``attrs`` under the
  argument's name (the "scalar binary" form, `npu_compiler/codegen_ops.py:386-388`);
* every other argument goes to ``attrs`` by schema name; dtypes are written as
  ``"float32"``-style strings, devices / layouts / memory formats as strings, and
  ``-1`` entries of ``size`` / ``shape`` lists are resolved from the node's output
  shape (the shapes are static);
* a node with a tuple result gets outputs ``<name>_out<i>`` and each
  ``operator.getitem`` becomes a ``<built-in function getitem>`` node over all of
  them with ``attrs.index`` (the reference's form, `subgraph_analyzer.py:395-409`);
* ``torch.no_grad()`` regions arrive as ``wrap_with_set_grad_enabled(False, submod,
  *args)``. When the region is HF's rotary embedding (``inv_freq`` times positions,
  ``cat``, ``cos`` / ``sin`` times one scaling constant, cast) it is written as one
  ``wrap_with_set_grad_enabled`` node over ``[inv_freq, position_ids]`` with two
  outputs and ``attrs.attention_scaling`` when the constant is not 1, which is how
  the reference's IR carries it; any other region is inlined op by op;
* ``aten._assert_tensor_metadata`` and other assertion nodes are dropped.

Placeholders of parameters and buffers become ``weights`` entries (only those
some node reads), keyed by their state-dict name with ``strip_prefix`` removed
(the reference's wrappers hold the model as ``self.model``, so its keys carry a
``model.`` prefix, `examples/run_qwen_graph.py:58-70`); ``weight_name_mapping``
maps placeholder → key. Tied parameters are one placeholder (export keeps one
name for a shared tensor).
"""

from __future__ import annotations

import operator
from typing import Any, Sequence

import torch

_DTYPE_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16",
                torch.float64: "float64", torch.int64: "int64", torch.int32: "int32", torch.int16: "int16",
                torch.int8: "int8", torch.uint8: "uint8", torch.bool: "bool"}

_DROP = {"aten._assert_tensor_metadata.default", "aten._assert_scalar.default",
         "aten.sym_constrain_range_for_size.default", "aten._assert_async.msg"}

# ops allowed inside a rotary region, besides the required matmul / cat / cos / sin
_ROTARY_OPS = {"aten.unsqueeze.default", "aten.to.dtype", "aten.to.dtype_layout", "aten.expand.default",
               "aten.matmul.default", "aten.transpose.int", "aten.cat.default", "aten.cos.default",
               "aten.sin.default", "aten.mul.Tensor", "aten._to_copy.default"} | _DROP


def _spec(name: str, val: torch.Tensor, producer: str | None = None, idx: int = 0) -> dict:
    d = {"name": name, "shape": [int(s) for s in val.shape], "dtype": _DTYPE_NAMES[val.dtype]}
    if producer is not None:
        d["producer_node"] = producer
        d["producer_output_idx"] = idx
    return d


def _attr_value(v: Any) -> Any:
    if isinstance(v, torch.dtype):
        return _DTYPE_NAMES[v]
    if isinstance(v, (torch.device, torch.layout, torch.memory_format)):
        return str(v)
    if isinstance(v, (list, tuple)):
        return [_attr_value(x) for x in v]
    if isinstance(v, (torch.SymInt, torch.SymFloat, torch.SymBool)):
        raise NotImplementedError("symbolic shapes are not supported: export with static shapes")
    return v


def _is_tensor_arg(t: str) -> bool:
    return t in ("Tensor", "Optional[Tensor]")


def _is_tensor_list_arg(t: str) -> bool:
    return t in ("List[Tensor]", "List[Optional[Tensor]]")


class _Emitter:
    def __init__(self) -> None:
        self.nodes: list[dict] = []
        self.used: set[str] = set()      # value names some emitted node reads
        self.specs: dict[str, dict] = {}  # value name -> tensor spec
        self._names: set[str] = set()

    def spec_of(self, node: torch.fx.Node, env: dict) -> dict:
        return dict(self.specs[env[node]])

    def fresh(self, base: str) -> str:
        name, k = base, 0
        while name in self._names:
            k += 1
            name = f"{base}_{k}"
        self._names.add(name)
        return name


def _rotary_scaling(gm: torch.fx.GraphModule) -> float | None:
    """The scaling constant if ``gm`` is HF's rotary-embedding region, else None."""
    ops, consts = [], []
    outs = None
    for n in gm.graph.nodes:
        if n.op == "call_function":
            name = str(n.target)
            if name not in _ROTARY_OPS:
                return None
            ops.append(name)
            if name == "aten.mul.Tensor":
                if not isinstance(n.args[1], (int, float)) or n.args[0].target not in (
                        torch.ops.aten.cos.default, torch.ops.aten.sin.default):
                    return None
                consts.append(float(n.args[1]))
        elif n.op == "placeholder":
            continue
        elif n.op == "output":
            outs = n.args[0]
        else:
            return None
    n_ph = sum(1 for n in gm.graph.nodes if n.op == "placeholder")
    need = {"aten.matmul.default", "aten.cat.default", "aten.cos.default", "aten.sin.default"}
    if n_ph != 2 or not need <= set(ops) or outs is None or len(outs) != 2:
        return None
    if len(set(consts)) > 1:
        return None
    return consts[0] if consts else 1.0


def _emit_graph(em: _Emitter, gm: torch.fx.GraphModule, env: dict[Any, Any], root: torch.fx.GraphModule,
                size_resolve: bool = True) -> Any:
    """Emit every call node of ``gm``; ``env`` maps fx nodes to IR value names (or, for
    tuple results, lists of names). Returns the output node's mapped value."""
    for n in gm.graph.nodes:
        if n.op in ("placeholder", "get_attr"):
            continue
        if n.op == "output":
            return [env.get(a) if isinstance(a, torch.fx.Node) else a for a in n.args[0]]
        tgt = n.target
        if tgt is operator.getitem:
            src, idx = n.args
            multi = env[src]
            name = em.fresh(n.name)
            val = n.meta["val"]
            srcs = multi["names"]
            out = _spec(name, val, name, 0)
            em.nodes.append({"name": name, "op_type": "<built-in function getitem>",
                             "inputs": [dict(s) for s in multi["specs"]],
                             "outputs": [out], "attrs": {"index": int(idx)}})
            em.used.update(srcs)
            em.specs[name] = out
            env[n] = name
            continue
        if str(tgt) == "wrap_with_set_grad_enabled":
            sub = getattr(root, n.args[1].target)
            tensor_args = list(n.args[2:])
            scaling = _rotary_scaling(sub)
            vals = n.meta["val"]
            if scaling is not None:
                name = em.fresh(n.name)
                outs = [_spec(f"{name}_out{i}", v, name, i) for i, v in enumerate(vals)]
                ins = [env[a] for a in tensor_args]
                specs = [em.spec_of(a, env) for a in tensor_args]
                em.used.update(ins)
                attrs = {} if scaling == 1.0 else {"attention_scaling": scaling}
                em.nodes.append({"name": name, "op_type": "wrap_with_set_grad_enabled", "inputs": specs,
                                 "outputs": outs, "attrs": attrs})
                for o in outs:
                    em.specs[o["name"]] = o
                env[n] = {"names": [o["name"] for o in outs], "specs": outs}
            else:   # inline the region
                sub_env: dict[Any, Any] = {}
                phs = [p for p in sub.graph.nodes if p.op == "placeholder"]
                for p, a in zip(phs, tensor_args):
                    sub_env[p] = env[a]
                res = _emit_graph(em, sub, sub_env, sub)
                env[n] = {"names": res, "specs": [dict(em.specs[r]) for r in res]}
            continue
        op_type = str(tgt)
        if op_type in _DROP:
            continue
        if not isinstance(tgt, torch._ops.OpOverload):
            raise NotImplementedError(f"cannot export node {n.name}: target {tgt!r}")
        name = em.fresh(n.name)
        val = n.meta["val"]
        inputs, attrs = [], {}
        args, kwargs = n.args, n.kwargs
        for i, a in enumerate(tgt._schema.arguments):
            if i < len(args) and not a.kwarg_only:
                v, given = args[i], True
            elif a.name in kwargs:
                v, given = kwargs[a.name], True
            else:
                v, given = None, False
            t = str(a.type)
            if not given:
                continue
            if _is_tensor_list_arg(t):
                for x in v:
                    inputs.append(em.spec_of(x, env))
                    em.used.add(env[x])
            elif _is_tensor_arg(t) and isinstance(v, torch.fx.Node):
                inputs.append(em.spec_of(v, env))
                em.used.add(env[v])
            elif _is_tensor_arg(t):
                attrs[a.name] = _attr_value(v)
            else:
                av = _attr_value(v)
                if size_resolve and a.name in ("size", "shape") and isinstance(av, list) and -1 in av \
                        and isinstance(val, torch.Tensor):
                    av = [int(s) for s in val.shape]
                attrs[a.name] = av
        if isinstance(val, (tuple, list)):
            outs = [_spec(f"{name}_out{i}", v, name, i) for i, v in enumerate(val)]
            env[n] = {"names": [o["name"] for o in outs], "specs": outs}
        else:
            outs = [_spec(name, val, name, 0)]
            env[n] = name
        for o in outs:
            em.specs[o["name"]] = o
        em.nodes.append({"name": name, "op_type": op_type, "inputs": inputs, "outputs": outs, "attrs": attrs})
    raise RuntimeError("graph has no output node")


def extract_ir(module: torch.nn.Module, example_inputs: Sequence[Any], model_name: str = "model",
               input_names: Sequence[str] | None = None, strip_prefix: str = "") -> dict:
    """Export ``module(*example_inputs)`` and return its IR dict (reference schema).

    ``example_inputs`` may live on the ``meta`` device (only shapes and dtypes are
    read). ``input_names`` renames the user inputs in order; ``strip_prefix`` is
    removed from the front of every state-dict key.
    """
    # traced with grad mode on: ``torch.no_grad()`` regions then stay visible as
    # ``wrap_with_set_grad_enabled`` nodes
    with torch.enable_grad():
        ep = torch.export.export(module, tuple(example_inputs), strict=False)
    gm = ep.graph_module
    sig = ep.graph_signature
    ph_nodes = {n.name: n for n in gm.graph.nodes if n.op == "placeholder"}
    env: dict[Any, Any] = {}
    em = _Emitter()
    graph_inputs, weights, mapping = [], [], {}
    kinds = {}
    user_i = 0
    for spec in sig.input_specs:
        node = ph_nodes[spec.arg.name]
        kind = spec.kind.name
        if kind == "USER_INPUT":
            name = input_names[user_i] if input_names is not None else spec.arg.name
            user_i += 1
            env[node] = name
            em.specs[name] = _spec(name, node.meta["val"])
            graph_inputs.append(dict(em.specs[name]))
            em._names.add(name)
        elif kind in ("PARAMETER", "BUFFER"):
            key = spec.target
            if strip_prefix and key.startswith(strip_prefix):
                key = key[len(strip_prefix):]
            env[node] = spec.arg.name
            em.specs[spec.arg.name] = _spec(spec.arg.name, node.meta["val"])
            kinds[spec.arg.name] = (key, node.meta["val"])
            em._names.add(spec.arg.name)
        else:
            raise NotImplementedError(f"input kind {kind} ({spec.arg.name}) is not supported")
    if input_names is not None and user_i != len(input_names):
        raise ValueError(f"{len(input_names)} input names for {user_i} user inputs")
    outs = _emit_graph(em, gm, env, gm)
    out_specs = []
    for spec, o in zip(sig.output_specs, outs):
        if spec.kind.name != "USER_OUTPUT":
            raise NotImplementedError(f"output kind {spec.kind.name} is not supported (in-place buffer update?)")
        if isinstance(o, dict):
            raise NotImplementedError("tuple-valued graph outputs are not supported")
        out_specs.append({k: em.specs[o][k] for k in ("name", "shape", "dtype")})
    for ph, (key, val) in kinds.items():
        if ph not in em.used:
            continue
        weights.append({"name": key, "shape": [int(s) for s in val.shape], "dtype": _DTYPE_NAMES[val.dtype]})
        mapping[ph] = key
    return {"model_name": model_name, "graph_inputs": graph_inputs, "graph_outputs": out_specs,
            "weights": weights, "weight_name_mapping": mapping, "nodes": em.nodes, "constants": {}}

