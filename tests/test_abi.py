"""ABI byte layout and exported symbols of the C boundary (CPU only)."""
import ctypes
import json
import os
import re
import subprocess

import helpers

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "abi_layout_ref.json")

# Layouts the reference headers cannot produce (kv_prefix.h's static asserts
# fail; sample.h / attention_decode.h include CUDA headers). Pinned by the
# packed/natural-alignment arithmetic of their field lists.
ARITHMETIC = {
    "KVPrefix.sizeof": 28, "KVPrefix.refcnt": 4, "KVPrefix.kv_block_offset": 8, "KVPrefix.token_len": 16,
    "KVPrefix.kv_block_count": 20, "KVPrefix.flags": 24,
    "KVBranch.sizeof": 36, "KVBranch.prefix_id": 8, "KVBranch.delta_kv_offset": 12, "KVBranch.delta_len": 20,
    "KVBranch.delta_block_count": 24, "KVBranch.state": 28, "KVBranch.flags": 32,
    "KVPrefixTable.sizeof": 606280, "KVPrefixTable.prefix_bitmap": 14336, "KVPrefixTable.branches": 14400,
    "KVPrefixTable.branch_bitmap": 604224, "KVPrefixTable.next_branch_id": 606272,
    "SampleState.sizeof": 48, "SampleState.temperature": 32, "SampleState.top_k": 36, "SampleState.top_p": 40,
    "SampleState.vocab_size": 44,
    "DecodeStepArgs.sizeof": 40, "DecodeStepArgs.seq_len": 16, "DecodeStepArgs.output_token_offset": 32,
    "DecodeStepResult.sizeof": 24, "DecodeStepResult.cycle_estimate": 16, "DecodeMicrokernelConfig.sizeof": 20,
}


def _runtime_layout():
    exe = helpers.build("tests/abi_probe.c")
    return json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)


def test_layout_matches_reference_headers():
    ref = json.load(open(GOLDEN))
    mine = _runtime_layout()
    assert len(ref) > 80
    mismatches = {k: (v, mine.get(k)) for k, v in ref.items() if mine.get(k) != v}
    assert not mismatches, mismatches


def test_layout_matches_appendix_arithmetic():
    mine = _runtime_layout()
    mismatches = {k: (v, mine.get(k)) for k, v in ARITHMETIC.items() if mine.get(k) != v}
    assert not mismatches, mismatches


def _declared_functions():
    names = set()
    for fn in sorted(os.listdir(helpers.INC)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(helpers.INC, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        # drop static inline bodies and macros
        text = re.sub(r"^#.*$", "", text, flags=re.M)
        for m in re.finditer(r"^(?!static|typedef|\s)([A-Za-z_][\w \*]*?)\b(\w+)\s*\(([^;{}]*)\)\s*;", text,
                             flags=re.M):
            names.add(m.group(2))
    return names


def test_library_exports_every_declared_function(rl):
    declared = _declared_functions()
    assert {"infer_submit_decode", "rl_hip_attn_decode", "kv_branch_total_offset", "rl_hip_sample",
            "hw_worker_sim_run", "arena_init"} <= declared
    lib = ctypes.CDLL(rl.LIB_PATH)
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing


def test_compute_entry_points_fail_loudly_without_device(rl):
    # No rl_hip_open in this process: every device entry point refuses.
    if rl.lib().rl_hip_is_open():
        return
    a = rl.AttnArgs()
    assert rl.lib().rl_hip_attn_decode(ctypes.byref(a)) == -1
    assert b"no device open" in rl.lib().rl_hip_last_error()
    s = rl.SampleArgs()
    assert rl.lib().rl_hip_sample(ctypes.byref(s)) == -1
    assert rl.lib().rl_hip_dev_alloc(64) is None
