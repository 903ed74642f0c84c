"""The Odin binding (odin-infer_amd/odin/engine.odin) declares everything the
reference's callers of the `infer` package use, with the reference's field
names, order and types, so those call sites compile against it unchanged.

No Odin compiler exists in this image, so this is a declaration-level check
of the binding's text.  The identifiers below are the complete set that the
reference's callers take from `infer` (every `infer.X` in the reference tree):
  oracle_harness/oracle.odin:182 Engine; :413-417 engine_load, Engine_Opts
    {max_ctx, use_metal, num_threads}; :422-423 engine_destroy,
    destroy_matmul_pool; :425 engine_config, Config.vocab_size (compared with
    an `int`, so the field must be `int`)
  oracle_harness/gen_self_fixture.odin:57-67 engine_load, Engine_Opts,
    engine_destroy, destroy_matmul_pool, engine_config
  doctor_harness/doctor.odin:218 DEFAULT_MAX_CONTEXT; :249-291 engine_load,
    engine_destroy, destroy_matmul_pool, engine_config, every Config field,
    engine_metal_ready
  sampler/sampler.odin:182 softmax
and the procedures of the reference's own engine file (infer/engine.odin:
7-60) and matmul pool (infer/matmul.odin:28-61).
"""
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINDING = os.path.join(REPO, "odin-infer_amd", "odin", "engine.odin")

CALLER_IDENTIFIERS = [
    "Engine", "Engine_Opts", "Config", "DEFAULT_MAX_CONTEXT", "engine_load", "engine_destroy", "engine_forward",
    "engine_config", "engine_metal_ready", "matmul_set_threads", "destroy_matmul_pool", "softmax",
]
# infer/engine.odin:7-11, in order
ENGINE_OPTS_FIELDS = [("max_ctx", "int"), ("use_metal", "bool"), ("num_threads", "int")]
# infer/model.odin:12-24, in order
CONFIG_FIELDS = [("dim", "int"), ("hidden_dim", "int"), ("n_layers", "int"), ("n_heads", "int"),
                 ("n_kv_heads", "int"), ("vocab_size", "int"), ("seq_len", "int"), ("max_seq", "int"),
                 ("head_dim", "int"), ("rope_freq", "f32"), ("rms_eps", "f32")]
# procedure signatures of the reference (parameter types, result types)
PROCS = {
    "engine_load": ("path: string, opts: Engine_Opts", "(Engine, bool)"),
    "engine_destroy": ("e: ^Engine", None),
    "engine_forward": ("e: ^Engine, token, pos: int", "[]f32"),
    "engine_config": ("e: ^Engine", "^Config"),
    "engine_metal_ready": ("e: ^Engine", "bool"),
    "matmul_set_threads": ("n: int", None),
    "destroy_matmul_pool": ("", None),
    "softmax": ("x: []f32", None),
}


def _text():
    text = open(BINDING).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.sub(r"//[^\n]*", "", text)


def _struct_fields(text, name):
    m = re.search(r"\b%s\s*::\s*struct\s*\{(.*?)\}" % name, text, flags=re.S)
    assert m, name
    return [(a, b) for a, b in re.findall(r"(\w+)\s*:\s*([\w^\[\]]+)\s*,", m.group(1))]


def test_binding_is_package_infer_with_foreign_import():
    text = _text()
    assert re.search(r"^package infer\b", text, flags=re.M)
    assert re.search(r'foreign import oi "system:oi_hip"', text)
    assert '@(default_calling_convention = "c")' in text


@pytest.mark.parametrize("ident", CALLER_IDENTIFIERS)
def test_caller_identifier_declared(ident):
    assert re.search(r"^%s\s*::" % re.escape(ident), _text(), flags=re.M), ident


def test_engine_opts_keeps_reference_fields_in_order():
    fields = _struct_fields(_text(), "Engine_Opts")
    assert fields[:len(ENGINE_OPTS_FIELDS)] == ENGINE_OPTS_FIELDS, fields
    assert ("use_hip", "bool") in fields


def test_config_fields_types_and_order():
    assert _struct_fields(_text(), "Config") == CONFIG_FIELDS


@pytest.mark.parametrize("name", sorted(PROCS))
def test_procedure_signatures(name):
    params, result = PROCS[name]
    m = re.search(r"^%s\s*::\s*proc\s*\(([^)]*)\)\s*(->\s*([^{]+?))?\s*\{" % name, _text(), flags=re.M)
    assert m, name
    assert m.group(1).strip() == params, (name, m.group(1))
    got = m.group(3).strip() if m.group(3) else None
    assert got == result, (name, got)


def test_default_max_context_value():
    # infer/model.odin:10
    assert re.search(r"^DEFAULT_MAX_CONTEXT\s*::\s*4096\b", _text(), flags=re.M)


def test_foreign_declarations_match_c_header():
    """Every foreign proc of the binding exists in include/oi.h with the same
    parameter count."""
    text = _text()
    block = re.search(r"foreign oi \{(.*?)\n\}", text, flags=re.S).group(1)
    header = open(os.path.join(REPO, "include", "oi.h")).read()
    header = re.sub(r"/\*.*?\*/", "", header, flags=re.S)
    protos = {m.group(1): m.group(2) for m in re.finditer(r"\b(oi_[a-z0-9_]+)\s*\(([^()]*)\)\s*;", header)}
    found = re.findall(r"(oi_\w+)\s*::\s*proc\s*\(([^)]*)\)", block)
    assert found
    for name, params in found:
        assert name in protos, name
        n_odin = 0 if not params.strip() else len(params.split(","))
        c = protos[name].strip()
        n_c = 0 if c in ("", "void") else c.count(",") + 1
        assert n_odin == n_c, (name, n_odin, n_c)
