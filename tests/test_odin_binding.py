"""The Odin bindings (odin-infer_amd/odin/infer/engine.odin, package infer;
odin-infer_amd/odin/qwen3_5/engine.odin, package qwen3_5) declare everything
the reference's callers of the `infer` and `qwen3_5` packages use, with the
reference's field names, order and types, so those call sites compile
against them unchanged (with -collection:infer= / -collection:qwen3_5= set to
odin-infer_amd/odin, the reference's `infer:infer` and `qwen3_5:qwen3_5`
imports resolve to them).

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

The callers of `qwen3_5` (serve_harness/serve.odin, imported as q35): :320
Engine; :440-458 engine_config and the Config fields vocab_size, dim,
hidden_dim, n_layers, n_full, n_linear, n_heads, n_kv_heads, head_dim,
seq_len, max_seq, and engine.metal_ready; :488-525, 889-994, 1085-1141,
1380-1421 engine_forward_batch, engine_forward, engine_reset_state,
engine_save_full_state, engine_restore_full_state; :1525-1548 engine_load
with Engine_Opts{max_ctx, use_metal, num_threads}, engine_destroy,
destroy_matmul_pool, engine_config, metal_ready.  Plus the package's own
public procedures (qwen3_5/engine.odin:7-174, kv_persist.odin:365-381,
infer/matmul.odin:28-61).
"""
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINDING = os.path.join(REPO, "odin-infer_amd", "odin", "infer", "engine.odin")
BINDING_Q35 = os.path.join(REPO, "odin-infer_amd", "odin", "qwen3_5", "engine.odin")

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


def _text(path=BINDING):
    text = open(path).read()
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


@pytest.mark.parametrize("path", [BINDING, BINDING_Q35])
def test_foreign_declarations_match_c_header(path):
    """Every foreign proc of the binding exists in include/oi.h with the same
    parameter count."""
    text = _text(path)
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


def test_infer_engine_has_metal_ready_field():
    # infer/engine.odin:13-16
    assert ("metal_ready", "bool") in _struct_fields(_text(), "Engine")


# ---------------------------------------------------------------- qwen3_5 --
Q35_IDENTIFIERS = [
    "Engine", "Engine_Opts", "Config", "Layer_Type", "DEFAULT_MAX_CONTEXT", "engine_load", "engine_destroy",
    "engine_forward", "engine_forward_batch", "engine_batch_max", "engine_config", "engine_reset_state",
    "engine_save_full_state", "engine_restore_full_state", "engine_save_spec_state", "engine_restore_spec_state",
    "engine_verify_batch", "engine_save_kv", "engine_load_kv", "matmul_set_threads", "destroy_matmul_pool",
]
# qwen3_5/engine.odin:7-11, in order (not infer's order)
Q35_OPTS_FIELDS = [("max_ctx", "int"), ("num_threads", "int"), ("use_metal", "bool")]
# qwen3_5/model.odin:20-45, in order
Q35_CONFIG_FIELDS = [
    ("dim", "int"), ("hidden_dim", "int"), ("n_layers", "int"), ("n_heads", "int"), ("n_kv_heads", "int"),
    ("head_dim", "int"), ("vocab_size", "int"), ("seq_len", "int"), ("max_seq", "int"), ("rms_eps", "f32"),
    ("rope_theta", "f32"), ("partial_rotary", "f32"), ("rotary_dim", "int"), ("lin_n_k_heads", "int"),
    ("lin_n_v_heads", "int"), ("lin_head_k_dim", "int"), ("lin_head_v_dim", "int"), ("lin_conv_kernel", "int"),
    ("full_attn_interval", "int"), ("layer_types", "[]Layer_Type"), ("n_full", "int"), ("n_linear", "int")]
# the fields serve_harness/serve.odin:447-458 reads
Q35_CONFIG_USED = ["vocab_size", "dim", "hidden_dim", "n_layers", "n_full", "n_linear", "n_heads", "n_kv_heads",
                   "head_dim", "seq_len", "max_seq"]
Q35_PROCS = {
    "engine_load": ("path: string, opts: Engine_Opts", "(Engine, bool)"),
    "engine_destroy": ("e: ^Engine", None),
    "engine_forward": ("e: ^Engine, token, pos: int", "[]f32"),
    "engine_forward_batch": ("e: ^Engine, tokens: []int, pos_start: int", "[]f32"),
    "engine_batch_max": ("", "int"),
    "engine_config": ("e: ^Engine", "^Config"),
    "engine_reset_state": ("e: ^Engine", None),
    "engine_save_full_state": ("e: ^Engine", "(kv_k: []u8, kv_v: []u8, conv: []u8, rec: []u8)"),
    "engine_restore_full_state": ("e: ^Engine, kv_k, kv_v, conv, rec: []u8", None),
    "engine_save_spec_state": ("e: ^Engine", "(conv: []u8, rec: []u8)"),
    "engine_restore_spec_state": ("e: ^Engine, conv: []u8, rec: []u8", None),
    "engine_verify_batch": ("e: ^Engine, tokens: []int, pos_start: int", "[]f32"),
    "engine_save_kv": ("e: ^Engine, path: string, n_valid_pos: int", "bool"),
    "engine_load_kv": ("e: ^Engine, path: string", "(int, bool)"),
    "matmul_set_threads": ("n: int", None),
    "destroy_matmul_pool": ("", None),
}


def test_q35_binding_is_package_qwen3_5_with_foreign_import():
    text = _text(BINDING_Q35)
    assert re.search(r"^package qwen3_5\b", text, flags=re.M)
    assert re.search(r'foreign import oi "system:oi_hip"', text)
    assert '@(default_calling_convention = "c")' in text


@pytest.mark.parametrize("ident", Q35_IDENTIFIERS)
def test_q35_identifier_declared(ident):
    assert re.search(r"^%s\s*::" % re.escape(ident), _text(BINDING_Q35), flags=re.M), ident


def test_q35_engine_opts_fields_in_order():
    fields = _struct_fields(_text(BINDING_Q35), "Engine_Opts")
    assert fields[:len(Q35_OPTS_FIELDS)] == Q35_OPTS_FIELDS, fields
    assert ("use_hip", "bool") in fields


def test_q35_engine_metal_ready_field():
    assert ("metal_ready", "bool") in _struct_fields(_text(BINDING_Q35), "Engine")


def test_q35_config_fields_types_and_order():
    fields = _struct_fields(_text(BINDING_Q35), "Config")
    assert fields == Q35_CONFIG_FIELDS
    assert set(Q35_CONFIG_USED) <= {f for f, _ in fields}


def test_q35_layer_type_enum_order():
    m = re.search(r"\bLayer_Type\s*::\s*enum\s*\{(.*?)\}", _text(BINDING_Q35), flags=re.S)
    assert m and re.findall(r"\w+", m.group(1)) == ["Full_Attention", "Linear_Attention"]


@pytest.mark.parametrize("name", sorted(Q35_PROCS))
def test_q35_procedure_signatures(name):
    params, result = Q35_PROCS[name]
    m = re.search(r"^%s\s*::\s*proc\s*\(([^)]*)\)\s*(->\s*([^{]+?))?\s*\{" % name, _text(BINDING_Q35), flags=re.M)
    assert m, name
    assert m.group(1).strip() == params, (name, m.group(1))
    got = m.group(3).strip() if m.group(3) else None
    assert got == result, (name, got)


def test_q35_default_max_context_value():
    # qwen3_5/model.odin:10
    assert re.search(r"^DEFAULT_MAX_CONTEXT\s*::\s*4096\b", _text(BINDING_Q35), flags=re.M)
