"""Write the reference generator's parameter names and shapes as a fixture,
read from its module definitions with ``ast`` (nothing of the reference is
imported or run).

    python tests/golden/make_param_names.py     # -> tests/golden/reference_param_names.json

The reference builds its generator as ``CausalLTXModel(CausalLTXModelConfig(
...))`` inside ``CausalLTX2DiffusionWrapper`` (state-dict prefix ``model.``;
taomate/inference/model_runtime.py:182-425, ltx_causal/wrapper.py:8-13).  This
script interprets the ``__init__`` bodies of the module classes in
ltx_causal/transformer/causal_model.py, causal_block.py, compat.py and
ltx_causal/attention/causal_attention.py for a given configuration: local
assignments, ``if`` branches and conditional expressions are evaluated,
``self.<name> = <module>`` registers a child, ``nn.Parameter(torch.empty(...))``
a parameter, and the torch leaves register what torch registers
(``nn.Linear``: weight [out, in] and bias [out]; ``nn.RMSNorm``: weight [dim];
``nn.LayerNorm``: weight and bias when elementwise_affine; ``nn.SiLU`` /
``nn.Identity``: nothing; ``nn.Sequential`` / ``nn.ModuleList``: children
"0", "1", ...).  Classes that are not ``nn.Module`` subclasses (the mask
builder) hold no parameters.

Three configurations are written, all with what load_model_generator
detects for the 22B V2 checkpoint and what taomate/inference/model.py:20-49
passes (no audio sink tokens, caption projection in the text connector):
  * "base": CausalLTXModelConfig's defaults otherwise (48 blocks, 4096 / 2048,
    no cross-attention AdaLN);
  * "production": plus gated attention, learned memory (kv side branch,
    every 4th block, 512 / 256, 8 heads) and the colour FiLM (hidden 256,
    condition 4 x 128);
  * "ltx23": "production" with the LTX-2.3 text cross-attention AdaLN.
Per configuration the fixture holds the top-level parameters and the
per-block parameters of a block without and with the memory adapters, and
which blocks have them, so the full name set is top-level plus
``transformer_blocks.<i>.<name>`` for every block.
"""
from __future__ import annotations

import ast
import json
import pathlib
import re
from collections import OrderedDict

REF = pathlib.Path("/root/reference")
FILES = [
    "ltx_causal/transformer/causal_model.py",
    "ltx_causal/transformer/causal_block.py",
    "ltx_causal/transformer/compat.py",
    "ltx_causal/attention/causal_attention.py",
    "ltx_causal/attention/mask_builder.py",
]
OUT = pathlib.Path(__file__).with_name("reference_param_names.json")

CONFIGS = {
    "base": dict(num_audio_sink_tokens=0, caption_proj_before_connector=True, cross_attention_adaln=False),
    "production": dict(num_audio_sink_tokens=0, caption_proj_before_connector=True, cross_attention_adaln=False,
                       apply_gated_attention=True, learned_memory_enabled=True,
                       learned_memory_mode="memory_kv_side_branch", learned_memory_layer_interval=4,
                       learned_memory_video_dim=512, learned_memory_audio_dim=256, learned_memory_heads=8,
                       learned_memory_color_film_enabled=True, learned_memory_color_condition_dim=4 * 128,
                       learned_memory_color_film_hidden_dim=256),
    # the LTX-2.3 base (ltx-2.3-22b-dev, README.md:72-123): text cross-attention
    # AdaLN, which load_model_generator detects from 9-row modulation tables
    "ltx23": dict(num_audio_sink_tokens=0, caption_proj_before_connector=True, cross_attention_adaln=True,
                  apply_gated_attention=True, learned_memory_enabled=True,
                  learned_memory_mode="memory_kv_side_branch", learned_memory_layer_interval=4,
                  learned_memory_video_dim=512, learned_memory_audio_dim=256, learned_memory_heads=8,
                  learned_memory_color_film_enabled=True, learned_memory_color_condition_dim=4 * 128,
                  learned_memory_color_film_hidden_dim=256),
}


class Module:
    def __init__(self, cls):
        self.cls = cls
        self.params = OrderedDict()
        self.children = OrderedDict()
        self.vals = {}

    def set(self, name, value):
        if isinstance(value, Module):
            self.children[name] = value
        elif isinstance(value, Param):
            self.params[name] = value.shape
        else:
            self.vals[name] = value

    def get(self, name):
        if name in self.children:
            return self.children[name]
        if name in self.vals:
            return self.vals[name]
        raise AttributeError(f"{self.cls}.{name}")

    def named(self, prefix=""):
        for k, v in self.params.items():
            yield prefix + k, list(v)
        for k, c in self.children.items():
            yield from c.named(prefix + k + ".")


class Param:
    def __init__(self, shape):
        self.shape = tuple(int(s) for s in shape)


class Shape(tuple):
    pass


class Obj:
    """A dataclass instance (configuration)."""

    def __init__(self, fields):
        self.__dict__.update(fields)


class Opaque:
    """An object without parameters (a non-module class, an enum member)."""


class Interp:
    def __init__(self):
        self.classes = {}
        for f in FILES:
            tree = ast.parse((REF / f).read_text(), filename=f)
            for node in tree.body:
                if isinstance(node, ast.ClassDef):
                    self.classes[node.name] = node

    # ---- classes ----
    def is_module(self, cdef):
        for b in cdef.bases:
            src = ast.unparse(b)
            if src in ("nn.Module", "torch.nn.Module"):
                return True
            if src in self.classes and self.is_module(self.classes[src]):
                return True
        return False

    def is_dataclass(self, cdef):
        return any(ast.unparse(d) in ("dataclass", "dataclasses.dataclass") for d in cdef.decorator_list)

    def dataclass_obj(self, name, args, kwargs):
        cdef = self.classes[name]
        fields = OrderedDict()
        for st in cdef.body:
            if isinstance(st, ast.AnnAssign) and isinstance(st.target, ast.Name):
                fields[st.target.id] = self.ev(st.value, {}) if st.value is not None else None
        names = list(fields)
        for n, a in zip(names, args):
            fields[n] = a
        for k, v in kwargs.items():
            if k not in fields:
                raise KeyError(f"{name} has no field {k}")
            fields[k] = v
        return Obj(fields)

    def construct(self, name, args, kwargs):
        leaf = self.leaf(name, args, kwargs)
        if leaf is not None:
            return leaf
        if name not in self.classes:
            raise KeyError(f"unknown class {name}")
        cdef = self.classes[name]
        if self.is_dataclass(cdef):
            return self.dataclass_obj(name, args, kwargs)
        if not self.is_module(cdef):
            return Opaque()
        init = next(n for n in cdef.body if isinstance(n, ast.FunctionDef) and n.name == "__init__")
        m = Module(name)
        env = {"self": m}
        a = init.args
        params = [p.arg for p in a.args][1:]
        defaults = a.defaults
        dstart = len(a.args) - len(defaults)
        for i, p in enumerate(a.args):
            if i == 0:
                continue
            if i - 1 < len(args):
                env[p.arg] = args[i - 1]
            elif p.arg in kwargs:
                env[p.arg] = kwargs[p.arg]
            elif i >= dstart:
                env[p.arg] = self.ev(defaults[i - dstart], env)
            else:
                raise TypeError(f"{name}: missing argument {p.arg}")
        for p, d in zip(a.kwonlyargs, a.kw_defaults):
            env[p.arg] = kwargs.get(p.arg, self.ev(d, env) if d is not None else None)
        if a.kwarg is not None:
            env[a.kwarg.arg] = {k: v for k, v in kwargs.items() if k not in params}
        self.exec_body(init.body, env)
        return m

    def leaf(self, name, args, kwargs):
        short = name.split(".")[-1] if name.startswith(("nn.", "torch.nn.")) else None
        if short is None:
            return None
        m = Module(name)
        if short == "Linear":
            fin, fout = args[0], args[1]
            bias = args[2] if len(args) > 2 else kwargs.get("bias", True)
            m.params["weight"] = (fout, fin)
            if bias:
                m.params["bias"] = (fout,)
        elif short == "RMSNorm":
            if kwargs.get("elementwise_affine", True):
                m.params["weight"] = (args[0],)
        elif short == "LayerNorm":
            if kwargs.get("elementwise_affine", True):
                m.params["weight"] = (args[0],)
                m.params["bias"] = (args[0],)
        elif short in ("SiLU", "Identity", "GELU"):
            pass
        elif short == "Sequential":
            for i, c in enumerate(args):
                m.children[str(i)] = c
        elif short == "ModuleList":
            for i, c in enumerate(args[0] if args else []):
                m.children[str(i)] = c
        elif short == "Parameter":
            return Param(args[0])
        else:
            raise KeyError(f"torch leaf {name} not modelled")
        return m

    # ---- statements ----
    def exec_body(self, body, env):
        for st in body:
            if isinstance(st, ast.Assign):
                val = self.ev(st.value, env)
                for t in st.targets:
                    self.assign(t, val, env)
            elif isinstance(st, ast.AnnAssign):
                if st.value is not None:
                    self.assign(st.target, self.ev(st.value, env), env)
            elif isinstance(st, ast.AugAssign):
                cur = self.ev(st.target, env)
                self.assign(st.target, self.binop(st.op, cur, self.ev(st.value, env)), env)
            elif isinstance(st, ast.If):
                self.exec_body(st.body if self.ev(st.test, env) else st.orelse, env)
            elif isinstance(st, ast.Raise):
                raise RuntimeError(f"reference raises: {ast.unparse(st)}")
            elif isinstance(st, (ast.Expr, ast.Pass, ast.Import, ast.ImportFrom)):
                continue    # super().__init__(), nn.init.*, docstrings: no parameters
            else:
                raise NotImplementedError(ast.unparse(st)[:80])

    def assign(self, t, val, env):
        if isinstance(t, ast.Name):
            env[t.id] = val
        elif isinstance(t, ast.Attribute) and isinstance(t.value, ast.Name) and t.value.id == "self":
            env["self"].set(t.attr, val)
        else:
            raise NotImplementedError(ast.unparse(t))

    # ---- expressions ----
    BUILTINS = {"int": int, "max": max, "min": min, "str": str, "bool": bool, "float": float, "range": range,
                "len": len, "None": None, "True": True, "False": False}

    def binop(self, op, a, b):
        return {ast.Add: lambda: a + b, ast.Sub: lambda: a - b, ast.Mult: lambda: a * b,
                ast.FloorDiv: lambda: a // b, ast.Div: lambda: a / b, ast.Mod: lambda: a % b}[type(op)]()

    def ev(self, n, env):
        if isinstance(n, ast.Constant):
            return n.value
        if isinstance(n, ast.Name):
            if n.id in env:
                return env[n.id]
            if n.id in self.BUILTINS:
                return self.BUILTINS[n.id]
            if n.id in self.classes:
                return ("class", n.id)
            raise NameError(n.id)
        if isinstance(n, ast.Attribute):
            src = ast.unparse(n)
            if src.startswith(("nn.", "torch.")):
                return ("class", src)
            if src.startswith("CausalRopeType."):
                return src
            base = self.ev(n.value, env)
            if isinstance(base, Module):
                return base.get(n.attr)
            return getattr(base, n.attr)
        if isinstance(n, ast.BinOp):
            return self.binop(n.op, self.ev(n.left, env), self.ev(n.right, env))
        if isinstance(n, ast.UnaryOp):
            v = self.ev(n.operand, env)
            return {ast.Not: lambda: not v, ast.USub: lambda: -v, ast.UAdd: lambda: +v}[type(n.op)]()
        if isinstance(n, ast.BoolOp):
            if isinstance(n.op, ast.And):
                v = True
                for x in n.values:
                    v = self.ev(x, env)
                    if not v:
                        return v
                return v
            v = False
            for x in n.values:
                v = self.ev(x, env)
                if v:
                    return v
            return v
        if isinstance(n, ast.Compare):
            left = self.ev(n.left, env)
            for op, c in zip(n.ops, n.comparators):
                right = self.ev(c, env)
                ok = {ast.Eq: lambda: left == right, ast.NotEq: lambda: left != right, ast.Lt: lambda: left < right,
                      ast.LtE: lambda: left <= right, ast.Gt: lambda: left > right, ast.GtE: lambda: left >= right,
                      ast.Is: lambda: left is right, ast.IsNot: lambda: left is not right,
                      ast.In: lambda: left in right, ast.NotIn: lambda: left not in right}[type(op)]()
                if not ok:
                    return False
                left = right
            return True
        if isinstance(n, ast.IfExp):
            return self.ev(n.body, env) if self.ev(n.test, env) else self.ev(n.orelse, env)
        if isinstance(n, (ast.Tuple, ast.List)):
            return [self.ev(x, env) for x in n.elts] if isinstance(n, ast.List) else tuple(self.ev(x, env) for x in n.elts)
        if isinstance(n, ast.Set):
            return {self.ev(x, env) for x in n.elts}
        if isinstance(n, ast.Dict):
            return {self.ev(k, env): self.ev(v, env) for k, v in zip(n.keys, n.values)}
        if isinstance(n, ast.ListComp):
            (gen,) = n.generators
            out = []
            for v in self.ev(gen.iter, env):
                e = dict(env)
                self.assign(gen.target, v, e)
                if all(self.ev(c, e) for c in gen.ifs):
                    out.append(self.ev(n.elt, e))
            return out
        if isinstance(n, ast.JoinedStr):
            return "<str>"
        if isinstance(n, ast.Call):
            fsrc = ast.unparse(n.func)
            args = []
            for a in n.args:
                if isinstance(a, ast.Starred):
                    args.extend(self.ev(a.value, env))
                else:
                    args.append(self.ev(a, env))
            kwargs = {k.arg: self.ev(k.value, env) for k in n.keywords if k.arg is not None}
            if fsrc in ("torch.empty", "torch.zeros", "torch.ones", "torch.randn"):
                return Shape(args[0] if len(args) == 1 and isinstance(args[0], (tuple, list)) else args)
            if fsrc == "replace":
                obj = Obj(dict(args[0].__dict__))
                obj.__dict__.update(kwargs)
                return obj
            if fsrc == "super":
                return Opaque()
            f = self.ev(n.func, env)
            if isinstance(f, tuple) and f and f[0] == "class":
                return self.construct(f[1], args, kwargs)
            if callable(f):
                return f(*args, **kwargs)
            raise NotImplementedError(fsrc)
        raise NotImplementedError(ast.dump(n)[:80])


def model_params(interp, overrides):
    cfg = interp.dataclass_obj("CausalLTXModelConfig", [], overrides)
    model = interp.construct("CausalLTXModel", [cfg], {})
    return OrderedDict(model.named()), cfg


def summarise(params, cfg):
    top, blocks = OrderedDict(), {}
    for name, shape in params.items():
        m = re.match(r"transformer_blocks\.(\d+)\.(.*)", name)
        if m:
            blocks.setdefault(int(m.group(1)), OrderedDict())[m.group(2)] = shape
        else:
            top[name] = shape
    kinds = {}
    adapter_blocks = []
    for i in sorted(blocks):
        key = "adapter" if any("memory_attn" in k or "color_film" in k for k in blocks[i]) else "plain"
        if key == "adapter":
            adapter_blocks.append(i)
        if key in kinds and kinds[key] != blocks[i]:
            raise RuntimeError(f"block {i} differs from the other {key} blocks")
        kinds[key] = blocks[i]
    return {"num_layers": len(blocks), "top": top, "block": kinds, "adapter_blocks": adapter_blocks,
            "video_dim": cfg.video_dim, "audio_dim": cfg.audio_dim, "in_channels": cfg.in_channels}


def main():
    interp = Interp()
    out = {"source": "ast of " + ", ".join(FILES) + " (CausalLTXModel.__init__ and the classes it builds); "
                     "state-dict keys carry the wrapper's 'model.' prefix",
           "configs": {}}
    for name, ov in CONFIGS.items():
        params, cfg = model_params(interp, ov)
        out["configs"][name] = dict(summarise(params, cfg), overrides=ov, total=len(params))
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    for name, c in out["configs"].items():
        print(name, c["total"], "parameters,", len(c["top"]), "top-level,",
              {k: len(v) for k, v in c["block"].items()}, "per block")


if __name__ == "__main__":
    main()
