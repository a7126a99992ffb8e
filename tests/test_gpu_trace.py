"""Trace replay on the GPU: workloads shaped like the official FlashInfer-Trace set
for this operator (token counts 1..901, local-expert offsets 0..224, the recorded
two-level routing bias), written as a trace set, loaded back and run through the
HIP operator; selection bit-exact and the output within atol=1e-2, rtol=2e-2 of
the CPU oracle."""
import pytest
import torch

import flashinfer_mlsys_amd as fm
from flashinfer_mlsys_amd import trace
from oracle import cpu_ref

from conftest import assert_close_bf16, write_trace_cases

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def trace_set(tmp_path_factory):
    root = tmp_path_factory.mktemp("trace")
    write_trace_cases(root)
    return str(root)


def test_trace_workloads_match_oracle(trace_set, weights, dev):
    _, jpath, blob = trace.trace_paths(trace_set)
    for w in trace.load_workloads(jpath):
        print(f"trace workload {w.uuid} T={w.T} offset={w.local_expert_offset}", flush=True)
        args = trace.load_inputs(w, trace_set, blob, device=dev, weights=weights[1])
        out = fm.run(*args)
        ids, _, _ = fm.route(args[0], args[1], args[9])
        cpu_args = [a.cpu() if isinstance(a, torch.Tensor) else a for a in args[:4]] + list(weights[0]) + args[8:]
        ref_ids = cpu_ref.sorted_selection(cpu_ref.route(cpu_args[0], cpu_args[1], w.routed_scaling_factor)[0])
        assert torch.equal(ids.cpu().long(), ref_ids.long()), w.uuid
        ref = cpu_ref.run(*cpu_args).float().numpy()
        assert_close_bf16(out.float().cpu().numpy(), ref, w.uuid)


@pytest.mark.parametrize("name", ["trace_t11948", "trace_t14107"])
def test_largest_official_sizes_through_the_trace_path(tmp_path, weights, dev, name):
    """The two largest official token counts and offsets (T=11,948 at offset 128,
    T=14,107 at offset 32) written as trace records, loaded back and replayed: the
    selection equals the reference's (golden fixture of the same inputs) bit for bit,
    and the output its rows within the bar."""
    from flashinfer_mlsys_amd import workloads as wl
    from conftest import bf16_bits_to_f32, load_golden
    w = wl.WORKLOADS[name]
    g = load_golden(name)
    uuid = f"mi355x-trace-{w.T}-{w.local_expert_offset}-0"
    write_trace_cases(tmp_path, [(uuid, w.T, w.local_expert_offset)])
    _, jpath, blob = trace.trace_paths(str(tmp_path))
    (tw,) = trace.load_workloads(jpath)
    assert tw.seed == w.seed
    args = trace.load_inputs(tw, str(tmp_path), blob, device=dev, weights=weights[1])
    for a, h in zip(args[:2], g["in_sha256"][:2]):
        assert wl.fingerprint(a) == str(h), "the trace records hold the workload's logits and bias"
    print(f"trace {uuid}", flush=True)
    ids, _, _ = fm.route(args[0], args[1], args[9])
    assert (ids.cpu().numpy() == g["sel_ids"].astype("int32")).all()
    out = fm.run(*args[:4], *weights[1], w.local_expert_offset, w.routed_scaling_factor)
    rows = g["out_rows"]
    assert_close_bf16(out.float().cpu().numpy()[rows], bf16_bits_to_f32(g["out_bf16"]), name)


def test_replay_runs_every_workload(trace_set, weights, dev):
    """The replay loop (as the command line runs it) gives the same outputs as direct calls."""
    _, jpath, blob = trace.trace_paths(trace_set)
    res = trace.replay(trace_set, iters=3, warmup=1, trials=1, device=dev)
    ws = trace.load_workloads(jpath)
    assert [r["uuid"] for r in res] == [w.uuid for w in ws]
    for r, w in zip(res, ws):
        args = trace.load_inputs(w, trace_set, blob, device=dev, weights=weights[1])
        assert torch.equal(r["output"].view(torch.int16), fm.run(*args).view(torch.int16)), w.uuid
        assert r["us_per_call"] > 0 and r["P"] > 0
