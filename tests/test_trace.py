"""FlashInfer-Trace loader (definition, workload JSONL, safetensors inputs) on the CPU.

The layout and record fields follow the reference's harness and notebook
(scripts/run_modal.py:139-155, input_analysis/input_check.ipynb cells 0-2,
reference moe/ref_moe.json:11-145 for the definition).
"""
import copy
import json
import os

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from flashinfer_mlsys_amd import trace, workloads as wl
from oracle import cpu_ref

from conftest import TRACE_CASES, trace_case_tensors, write_trace_cases


def _fake_weights():
    """Right-shaped, uninitialised expert weights (the loader only checks shapes and dtypes)."""
    return (torch.empty((32, 4096, 7168), dtype=torch.float8_e4m3fn), torch.empty((32, 32, 56)),
            torch.empty((32, 7168, 2048), dtype=torch.float8_e4m3fn), torch.empty((32, 56, 16)))


def test_definition_is_the_operators():
    d = trace.definition_dict()
    trace.check_definition(json.loads(json.dumps(d)))
    assert d["name"] == "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048"
    assert [n for n in d["inputs"]] == ["routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
                                        "gemm1_weights", "gemm1_weights_scale", "gemm2_weights",
                                        "gemm2_weights_scale", "local_expert_offset", "routed_scaling_factor"]
    assert d["inputs"]["hidden_states_scale"]["shape"] == ["num_hidden_blocks", "seq_len"]  # transposed scales
    assert d["axes"]["gemm1_out_size"]["value"] == 2 * d["axes"]["intermediate_size"]["value"]


REFERENCE_DEFINITION = "/root/reference/reference moe/ref_moe.json"


def test_reference_definition_accepted():
    """The reference's own definition file (reference moe/ref_moe.json:11-145) passes
    check_definition unchanged, and agrees with definition_dict() on every field the
    check reads."""
    if not os.path.exists(REFERENCE_DEFINITION):
        pytest.skip(f"{REFERENCE_DEFINITION} is not on this host (the reference tree is read here only)")
    with open(REFERENCE_DEFINITION) as f:
        ref = json.load(f)
    trace.check_definition(ref)
    mine = trace.definition_dict()
    assert ref["name"] == mine["name"]
    assert list(ref["inputs"]) == list(mine["inputs"])
    for n in mine["inputs"]:
        assert (ref["inputs"][n]["shape"], ref["inputs"][n]["dtype"]) == \
            (mine["inputs"][n]["shape"], mine["inputs"][n]["dtype"]), n
    for k, v in mine["axes"].items():
        assert ref["axes"][k]["type"] == v["type"], k
        if v["type"] == "const":
            assert ref["axes"][k]["value"] == v["value"], k
    broken = copy.deepcopy(ref)
    broken["inputs"]["hidden_states_scale"]["shape"] = ["seq_len", "num_hidden_blocks"]
    with pytest.raises(trace.TraceFormatError):
        trace.check_definition(broken)


@pytest.mark.parametrize("edit", [
    lambda d: d.update(name="other_op"),
    lambda d: d["axes"]["hidden_size"].update(value=4096),
    lambda d: d["axes"]["seq_len"].update(type="const"),
    lambda d: d["inputs"]["routing_bias"].update(dtype="float32"),
    lambda d: d["inputs"]["hidden_states_scale"].update(shape=["seq_len", "num_hidden_blocks"]),
    lambda d: d["inputs"].pop("routing_bias"),
    lambda d: d["outputs"]["output"].update(dtype="float32"),
])
def test_definition_mismatch_rejected(edit):
    d = copy.deepcopy(trace.definition_dict())
    edit(d)
    with pytest.raises(trace.TraceFormatError):
        trace.check_definition(d)


def test_write_then_load_roundtrip(tmp_path):
    cases = TRACE_CASES[:3]
    write_trace_cases(tmp_path, cases)
    dpath, jpath, blob = trace.trace_paths(str(tmp_path))
    trace.load_definition(dpath)
    ws = trace.load_workloads(jpath)
    assert [(w.uuid, w.T, w.local_expert_offset, w.routed_scaling_factor) for w in ws] == \
        [(u, T, off, 2.5) for u, T, off in cases]
    for w, (uuid, T, _) in zip(ws, cases):
        assert w.inputs["routing_logits"]["type"] == "safetensors"
        assert w.inputs["hidden_states"] == {"type": "random"}
        args = trace.load_inputs(w, str(tmp_path), weights=_fake_weights())
        lg, b = trace_case_tensors(uuid, T)
        assert torch.equal(args[0], lg) and torch.equal(args[1].view(torch.int16), b.view(torch.int16))
        # generated hidden states: the benchmark's quantised N(0,1) rows from the uuid seed
        _, _, hs, hss = wl.make_activations(T, w.seed)
        assert wl.fingerprint(args[2]) == wl.fingerprint(hs) and torch.equal(args[3], hss)
        assert args[8] == w.local_expert_offset and isinstance(args[8], int)
        assert args[9] == 2.5 and isinstance(args[9], float)


def test_reference_record_layout_and_path_resolution(tmp_path):
    """A record as the reference's files have it: the safetensors path relative to the
    trace-set root, or an absolute path from another machine whose file now sits in
    the blob directory, and records of other definitions in the same file."""
    _, jpath, blob = trace.trace_paths(str(tmp_path))
    os.makedirs(os.path.dirname(jpath))
    os.makedirs(blob)
    T = 5
    lg = torch.randn(T, 256)
    b = torch.full((256,), 4.9375, dtype=torch.bfloat16)
    save_file({"routing_logits": lg, "routing_bias": b}, os.path.join(blob, "abc.safetensors"))
    rel = os.path.relpath(os.path.join(blob, "abc.safetensors"), tmp_path)

    def rec(uuid, path, definition=trace.DEFINITION_NAME):
        st = {"type": "safetensors", "path": path}
        return {"definition": definition, "workload": {"uuid": uuid, "axes": {"seq_len": T}, "inputs": {
            "routing_logits": dict(st, tensor_key="routing_logits"), "routing_bias": dict(st, tensor_key="routing_bias"),
            "hidden_states": {"type": "random"}, "hidden_states_scale": {"type": "random"},
            "gemm1_weights": {"type": "random"}, "gemm1_weights_scale": {"type": "random"},
            "gemm2_weights": {"type": "random"}, "gemm2_weights_scale": {"type": "random"},
            "local_expert_offset": {"type": "scalar", "value": 192},
            "routed_scaling_factor": {"type": "scalar", "value": 2.5}}}}

    with open(jpath, "w") as f:
        f.write(json.dumps(rec("u-rel", "./" + rel)) + "\n\n")
        f.write(json.dumps(rec("u-abs", "/home/someone/trace/blob/workloads/moe/x/abc.safetensors")) + "\n")
        f.write(json.dumps(rec("u-other", "./nowhere", definition="another_op")) + "\n")
    ws = trace.load_workloads(jpath)
    assert [w.uuid for w in ws] == ["u-rel", "u-abs"]
    for w in ws:
        args = trace.load_inputs(w, str(tmp_path), weights=_fake_weights())
        assert torch.equal(args[0], lg) and args[8] == 192


def _record(**over):
    inputs = {"local_expert_offset": {"type": "scalar", "value": 0},
              "routed_scaling_factor": {"type": "scalar", "value": 2.5}}
    w = {"uuid": "x", "axes": {"seq_len": 3}, "inputs": inputs}
    for k, v in over.items():
        if k in ("uuid", "axes"):
            w[k] = v
        else:
            inputs[k] = v
    return {"workload": w}


@pytest.mark.parametrize("obj", [
    _record(uuid=""),
    _record(axes={"seq_len": -1}),
    _record(axes={"seq_len": 2.5}),
    _record(axes={"seq_len": 3, "hidden_size": 4096}),
    _record(routing_logits={"type": "zeros"}),
    _record(routing_logits={"type": "scalar", "value": 1.0}),
    _record(local_expert_offset={"type": "random"}),
    _record(local_expert_offset={"type": "scalar", "value": 1.5}),
    _record(routing_bias={"type": "safetensors"}),
    _record(not_an_input={"type": "random"}),
    {"workload": {"uuid": "x", "axes": {"seq_len": 3}, "inputs": {}}},
])
def test_bad_records_rejected(obj):
    with pytest.raises(trace.TraceFormatError):
        trace.parse_workload(obj)


def test_bad_tensors_rejected(tmp_path):
    blob = str(tmp_path)
    save_file({"routing_logits": torch.randn(3, 256, dtype=torch.float16),
               "short": torch.randn(2, 256)}, os.path.join(blob, "f.safetensors"))
    st = lambda key: {"type": "safetensors", "path": "f.safetensors", "tensor_key": key}  # noqa: E731
    cases = [
        (_record(routing_logits=st("routing_logits")), trace.TraceFormatError),   # fp16, not fp32
        (_record(routing_logits=st("short")), trace.TraceFormatError),            # [2, 256] for seq_len 3
        (_record(routing_logits=st("missing")), trace.TraceFormatError),          # no such key
        (_record(routing_logits={"type": "safetensors", "path": "none.safetensors"}), FileNotFoundError),
    ]
    for obj, err in cases:
        w = trace.parse_workload(obj)
        with pytest.raises(err):
            trace.load_inputs(w, blob, blob_dir=blob, weights=_fake_weights())


def test_not_json_rejected(tmp_path):
    p = tmp_path / "w.jsonl"
    p.write_text('{"workload": {"uuid": "a", "axes": {"seq_len": 1}, "inputs": {}}\n{oops\n')
    with pytest.raises(trace.TraceFormatError):
        trace.load_workloads(str(p))


def test_trace_cases_are_well_posed():
    """Every trace case has a local pair and selection margins of at least 8 fp32
    ulps under the oracle's routing, so the GPU replay's selection can be compared
    bit for bit (a gap of a few ulps could flip with the last bit of exp)."""
    for uuid, T, offset in TRACE_CASES:
        lg, b = trace_case_tensors(uuid, T)
        g, e = cpu_ref.selection_margins(lg, b)
        assert min(g, e) >= 8, (uuid, g, e)
        ids = cpu_ref.route(lg, b, 2.5)[0]
        assert int(((ids >= offset) & (ids < offset + 32)).sum()) > 0, uuid
        vals = np.unique(b.float().numpy())
        assert set(vals.tolist()) <= {4.9375, 4.96875}


def test_trace_cases_cover_every_official_workload():
    """The trace cases plus the two largest official workloads (trace_t11948,
    trace_t14107) are exactly the 19 official (T, offset) pairs."""
    from conftest import OFFICIAL_PAIRS
    pairs = [(T, off) for _, T, off in TRACE_CASES]
    pairs += [(wl.WORKLOADS[n].T, wl.WORKLOADS[n].local_expert_offset) for n in ("trace_t11948", "trace_t14107")]
    assert len(OFFICIAL_PAIRS) == 19 and sorted(pairs) == sorted(OFFICIAL_PAIRS)
    for uuid, T, off in TRACE_CASES:
        assert uuid.startswith(f"mi355x-trace-{T}-{off}-")
