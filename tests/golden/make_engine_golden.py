"""Write tests/golden/engine_0p8b.npz from the reference CpuEngine (built from
the reference sources into oracle/_ref) running the random-init 0.8B Q35H128
artifact that q35_write_random_artifact writes for (SEED, STD) below.

Two record sets:
  forced_*  teacher-forced: each of BATCH rows has a 1-token prompt and
            forced_output_tokens = the rest of a random sequence
            (cpu_engine.h:108), so every later token runs the batched decode
            path (advance_batch -> forward_batch) and the raw logits after each
            token are reported: the 8 largest of each position and the logits
            at PROBES fixed vocabulary indices, once per Q8_0 backend in
            BACKENDS (auto = the host's best ISA, scalar, avx2). The spread
            between the reference's own backends is the yardstick for
            whole-model logit parity: activation quantization rounds FP16
            scales, so last-ulp differences in a reduction move whole
            32-value blocks and the reference disagrees with itself across ISAs.
  greedy_*  free greedy decode from PROMPT-token prompts (the reference
            prefills those with its chunked batch forward), tokens and top-8
            logits of every generated position.

Run in the container that has the reference checkout:
    make -C oracle ref && python tests/golden/make_engine_golden.py [g16q8]
With g16q8 the artifact carries the optional encodings (G16 tied head,
Q8_0 gate rows; q35_write_random_artifact_ex) and the records go to
engine_0p8b_g16q8.npz (auto and scalar backends only).
The tests regenerate the same artifact (the generator is deterministic and
host-only) and compare against these vectors.
"""
from __future__ import annotations

import ctypes
import json
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import q35_oracle as orc  # noqa: E402

SEED, STD = 1, 0.02
BATCH, SEQ = 4, 24            # teacher-forced sequences
PROBES = 512
BACKENDS = (0, 1, 2)          # Q8_0Backend auto_select, scalar, avx2 (q8_0.h:23-31)
PROMPT, NEW = 16, 8           # free greedy


def run(model_dir, art, prompts, new, forced=None, backend=0, probe=None):
    b = prompts.shape[0]
    out = np.zeros((b, new), np.int32)
    top_v = np.zeros((b, new, 8), np.float32)
    top_i = np.zeros((b, new, 8), np.int32)
    ms = ctypes.c_double()
    err = ctypes.create_string_buffer(512)
    pv = np.zeros((b, new, 0 if probe is None else probe.size), np.float32)
    orc.ref().ref_engine_set_probe(None if probe is None else probe.ctypes.data, 0 if probe is None else probe.size,
                                   pv.ctypes.data)
    rc = orc.ref().ref_engine_greedy(os.fsencode(model_dir), os.fsencode(art), 8, backend, prompts.ctypes.data,
                                     prompts.shape[1], b, new, 1.0,
                                     None if forced is None else forced.ctypes.data, out.ctypes.data,
                                     top_v.ctypes.data, top_i.ctypes.data, ctypes.byref(ms), err, 512)
    orc.ref().ref_engine_set_probe(None, 0, None)
    assert rc == 0, err.value
    return out, top_v, top_i, pv


def main():
    import __graft_entry__ as entry
    import bench

    variant = sys.argv[1] if len(sys.argv) > 1 else "q4"
    assert variant in ("q4", "g16q8")
    alt = variant == "g16q8"
    backends = BACKENDS[:2] if alt else BACKENDS

    q = entry.load()
    assert orc.ref_available(), "build oracle/_ref first: make -C oracle ref"
    d, sched = q.model_dims(0)
    tmp = tempfile.mkdtemp(prefix="q35_golden_")
    art = os.path.join(tmp, "model.q35h128")
    q.write_random_artifact(art, d, sched, seed=SEED, weight_std=STD, head_g16=alt, q8_gates=alt)
    with open(os.path.join(tmp, "config.json"), "w") as f:
        json.dump(bench.CONFIG_08B, f)
    rng = np.random.default_rng(77)
    seq = rng.integers(0, d.vocab, size=(BATCH, SEQ)).astype(np.int32)
    forced = np.ascontiguousarray(seq[:, 1:])
    probe = np.sort(np.random.default_rng(99).choice(d.vocab, PROBES, replace=False)).astype(np.int32)
    rec = {}
    for bk in backends:
        out, fv, fi, pv = run(tmp, art, np.ascontiguousarray(seq[:, :1]), SEQ - 1, forced, bk, probe)
        assert np.array_equal(out, forced)
        rec.update({f"forced_b{bk}_top_values": fv, f"forced_b{bk}_top_index": fi, f"forced_b{bk}_probe": pv})
    for bk in backends[1:]:
        diff = np.abs(rec[f"forced_b{bk}_probe"] - rec["forced_b0_probe"])
        print(f"backend {bk} vs auto: probe logits max-abs {diff.max():.4f}, mean-abs {diff.mean():.5f}")
    prompts = rng.integers(0, d.vocab, size=(BATCH, PROMPT)).astype(np.int32)
    gt, gv, gi, _ = run(tmp, art, prompts, NEW)
    assert np.array_equal(gt, gi[:, :, 0]), "greedy token is the top logit at penalty 1"
    name = "engine_0p8b_g16q8.npz" if alt else "engine_0p8b.npz"
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), name),
                        seed=np.array([SEED]), weight_std=np.array([STD], np.float32),
                        forced_sequence=seq, probe_index=probe, backends=np.array(backends), **rec,
                        greedy_prompts=prompts, greedy_tokens=gt, greedy_top_values=gv, greedy_top_index=gi)
    os.remove(art)
    fv = rec["forced_b0_top_values"]
    print("teacher-forced top-1 margins min", float(np.min(fv[:, :, 0] - fv[:, :, 1])))


if __name__ == "__main__":
    main()
