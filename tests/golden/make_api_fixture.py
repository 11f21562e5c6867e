"""Write tests/golden/reference_api.json: the reference's solver API as its
Stage-A/B callers use it, read from the reference sources with ``ast``
(the reference is parsed as text, never imported or run).

Recorded:

* ``imports``: every ``from .<module> import <name>`` in the caller files,
  for the modules this build provides (capture, gptq, grid, packing,
  artifacts);
* ``defs``: for each such name, its definition in the reference module --
  a function's parameters (name, kind, default as source text), a class's
  ``__init__`` parameters, public methods and (for dataclasses) fields, or
  "constant";
* ``uses``: attribute names the callers read on objects of those classes
  (the capture manager, its stashes and tasks, the artifact writer and
  reader), found from constructor assignments, annotations and the
  ``<manager>.stashes[...]`` pattern.

Usage: python tests/golden/make_api_fixture.py [/root/reference]
"""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

CALLERS = ("sequential.py", "calibrate.py", "dflash2_calibrate.py", "pack.py", "stream_pack.py",
           "validate_artifacts.py", "qat.py", "dflash2_distill.py")
PROVIDED = ("capture", "gptq", "grid", "packing", "artifacts")
TRACKED = ("CaptureManager", "LinearTask", "FusedExpertTask", "ArtifactWriter", "ArtifactReader")
# unannotated parameters (and ``self.<name>`` attributes) of the callers that
# hold these objects
PARAM_NAMES = {"capture_mgr": "CaptureManager", "writer": "ArtifactWriter",
               "reader": "ArtifactReader", "reader_for_resume": "ArtifactReader"}


def _params(fn: ast.FunctionDef, src: str) -> list[dict]:
    a = fn.args
    out = []
    pos = a.posonlyargs + a.args
    defaults = [None] * (len(pos) - len(a.defaults)) + list(a.defaults)
    for arg, d in zip(pos, defaults):
        out.append({"name": arg.arg, "kind": "positional",
                    "default": None if d is None else ast.get_source_segment(src, d)})
    if a.vararg:
        out.append({"name": a.vararg.arg, "kind": "var_positional", "default": None})
    for arg, d in zip(a.kwonlyargs, a.kw_defaults):
        out.append({"name": arg.arg, "kind": "keyword_only",
                    "default": None if d is None else ast.get_source_segment(src, d)})
    if a.kwarg:
        out.append({"name": a.kwarg.arg, "kind": "var_keyword", "default": None})
    return out


def _definition(tree: ast.Module, src: str, name: str) -> dict:
    for node in tree.body:
        if isinstance(node, ast.FunctionDef) and node.name == name:
            return {"kind": "function", "params": _params(node, src), "line": node.lineno}
        if isinstance(node, ast.ClassDef) and node.name == name:
            methods, fields = {}, []
            is_dc = any((isinstance(d, ast.Name) and d.id == "dataclass") or
                        (isinstance(d, ast.Call) and getattr(d.func, "id", "") == "dataclass")
                        for d in node.decorator_list)
            for item in node.body:
                if isinstance(item, ast.FunctionDef) and (item.name == "__init__"
                                                          or not item.name.startswith("_")):
                    is_prop = any(isinstance(d, ast.Name) and d.id == "property"
                                  for d in item.decorator_list)
                    methods[item.name] = {"property": is_prop,
                                          "params": _params(item, src)}
                if is_dc and isinstance(item, ast.AnnAssign) and isinstance(item.target, ast.Name):
                    fields.append(item.target.id)
            return {"kind": "class", "methods": methods, "dataclass_fields": fields,
                    "line": node.lineno}
        if isinstance(node, (ast.Assign, ast.AnnAssign)):
            targets = node.targets if isinstance(node, ast.Assign) else [node.target]
            if any(isinstance(t, ast.Name) and t.id == name for t in targets):
                return {"kind": "constant", "line": node.lineno}
    raise KeyError(name)


class _Uses(ast.NodeVisitor):
    """Attribute names read on objects of the tracked classes."""

    def __init__(self):
        self.scopes = [{}]
        self.uses: dict[str, set[str]] = {}

    def _cls_of(self, node):
        if isinstance(node, ast.Name):
            for scope in reversed(self.scopes):
                if node.id in scope:
                    return scope[node.id]
        if (isinstance(node, ast.Attribute) and isinstance(node.value, ast.Name)
                and node.value.id == "self" and node.attr in PARAM_NAMES):
            return PARAM_NAMES[node.attr]
        if (isinstance(node, ast.Subscript) and isinstance(node.value, ast.Attribute)
                and node.value.attr == "stashes"
                and self._cls_of(node.value.value) == "CaptureManager"):
            return "Stash"
        return None

    def visit_FunctionDef(self, node):
        scope = {}
        for arg in node.args.posonlyargs + node.args.args + node.args.kwonlyargs:
            ann = arg.annotation
            if isinstance(ann, ast.Name) and ann.id in TRACKED:
                scope[arg.arg] = ann.id
            elif arg.arg in PARAM_NAMES:
                scope[arg.arg] = PARAM_NAMES[arg.arg]
        self.scopes.append(scope)
        self.generic_visit(node)
        self.scopes.pop()

    def visit_Assign(self, node):
        v = node.value
        if isinstance(v, ast.Call) and isinstance(v.func, ast.Name) and v.func.id in TRACKED:
            for t in node.targets:
                if isinstance(t, ast.Name):
                    self.scopes[-1][t.id] = v.func.id
        self.generic_visit(node)

    def visit_For(self, node):
        # for task in mgr.linear_tasks / mgr.fused_tasks
        it = node.iter
        if (isinstance(node.target, ast.Name) and isinstance(it, ast.Attribute)
                and self._cls_of(it.value) == "CaptureManager"
                and it.attr in ("linear_tasks", "fused_tasks")):
            self.scopes[-1][node.target.id] = ("LinearTask" if it.attr == "linear_tasks"
                                               else "FusedExpertTask")
        self.generic_visit(node)

    def visit_Attribute(self, node):
        cls = self._cls_of(node.value)
        if cls is not None:
            self.uses.setdefault(cls, set()).add(node.attr)
        self.generic_visit(node)


def main(ref_root: str) -> None:
    pkg = Path(ref_root) / "mlx_gptq"
    imports, defs = [], {}
    trees = {m: (ast.parse((pkg / f"{m}.py").read_text()), (pkg / f"{m}.py").read_text())
             for m in PROVIDED}
    uses = _Uses()
    for caller in CALLERS:
        src = (pkg / caller).read_text()
        tree = ast.parse(src)
        for node in ast.walk(tree):
            if isinstance(node, ast.ImportFrom) and node.level == 1 and node.module in PROVIDED:
                for alias in node.names:
                    imports.append({"caller": f"mlx_gptq/{caller}:{node.lineno}",
                                    "module": node.module, "name": alias.name})
                    key = f"{node.module}.{alias.name}"
                    if key not in defs:
                        mt, ms = trees[node.module]
                        defs[key] = _definition(mt, ms, alias.name)
        uses.visit(tree)
    # classes reached through the capture manager's attributes
    for cls, mod in (("LinearTask", "capture"), ("FusedExpertTask", "capture"),
                     ("Stash", "capture")):
        key = f"{mod}.{cls}"
        if key not in defs:
            mt, ms = trees[mod]
            defs[key] = _definition(mt, ms, cls)
    out = {
        "source": "reference mlx_gptq callers, parsed with ast (not imported)",
        "imports": imports,
        "defs": defs,
        "uses": {k: sorted(v) for k, v in sorted(uses.uses.items())},
    }
    dst = Path(__file__).with_name("reference_api.json")
    dst.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {dst}: {len(imports)} imports, {len(defs)} definitions")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
