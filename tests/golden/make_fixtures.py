#!/usr/bin/env python3
"""Writes the committed golden fixtures of tests/golden/.

Reference-produced (needs oracle/_ref, built from /root/reference by
oracle/build_ref.sh):
  ref_gaussian_codebook.txt  stdout of the reference's src/gaussian_codebook.cpp
                             (its own main(), :87-96): the 8-level Lloyd-Max
                             design behind the K3 codebook literals.
  ref_layouts.txt            the reference's make_tq_turbo_mse_page_layout
                             (src/tq_turbo_mse_layout.cpp:7-28) over 144
                             configs, via oracle/ref_layout_driver.cpp.
  ref_legacy_layouts.txt     every field of the reference's make_tq_page_layout
                             (src/tq_layout.cpp:8-36) and
                             make_tq_dense_page_layout (src/tq_dense_layout.cpp)
                             over 288 configs (FP16 and FP32 scales) and the
                             configs the legacy factory rejects, via
                             oracle/ref_legacy_layout_driver.cpp.

Oracle-produced (seeded inputs, this build's CPU restatement as the checker;
they pin the oracle against regressions and give the GPU tests fixed data):
  prod_n37_h2_d128.npz / mse_n37_h2_d128.npz
      key, value [37,2,128] fp16 bits (seed 900), slots (5-page pool, pages
      in seeded order, seed 901), query [8,2,128] fp16 bits (16 q heads,
      seed 902) -> pool bytes after pack, dequant K/V fp16 bits, logits
      (turbo_prod), attention in fp64 and with the reference kernel's fp32
      algorithm.

Generator records:
  synthetic_sha256.json      SHA-256 of the synthetic-input spec's tensors
                             (tests/test_synthetic.py: spec_inputs), so a
                             change of the generator or of numpy's math shows.

Usage: python tests/golden/make_fixtures.py
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle.oracle import load  # noqa: E402
from turborag_amd.synthetic import (as_u16, gqa_rows, kv_tokens_major,  # noqa: E402
                                    permuted_slots, query)

N, H, D, B, PAGES = 37, 2, 128, 16, 5


def reference_outputs() -> None:
    ref = ROOT / "oracle" / "_ref"
    for exe, name in (("gaussian_codebook", "ref_gaussian_codebook.txt"),
                      ("ref_layouts", "ref_layouts.txt"),
                      ("ref_legacy_layouts", "ref_legacy_layouts.txt")):
        path = ref / exe
        if not path.exists():
            raise SystemExit(f"{path} missing: run oracle/build_ref.sh first")
        out = subprocess.run([str(path)], capture_output=True, text=True, check=True).stdout
        (HERE / name).write_text(out)
        print(f"wrote {name} ({len(out)} B)")


def inputs():
    k, v = kv_tokens_major(N, H, D, seed=900)
    slots = permuted_slots(N, B, seed=901, num_pages=PAGES).numpy()
    q = gqa_rows(query(16, D, seed=902), H)
    return as_u16(k), as_u16(v), slots, as_u16(q)


def oracle_fixtures() -> None:
    orc = load()
    k, v, slots, q = inputs()
    pool = orc.prod_pack(k, v, slots, PAGES, B)
    dk, dv = orc.prod_dequant(pool, slots, H, D, B)
    np.savez_compressed(
        HERE / "prod_n37_h2_d128.npz", key=k, value=v, slots=slots, query=q, pool=pool,
        dequant_key=dk, dequant_value=dv, logits=orc.prod_logits(q, pool, slots, B),
        attention_f64=orc.prod_attention_f64(q, pool, slots, B),
        attention_f32=orc.prod_attention_f32(q, pool, slots, B))
    pool = orc.mse_pack(k, v, slots, PAGES, B)
    dk, dv = orc.mse_dequant(pool, slots, H, D, B)
    np.savez_compressed(
        HERE / "mse_n37_h2_d128.npz", key=k, value=v, slots=slots, query=q, pool=pool,
        dequant_key=dk, dequant_value=dv,
        attention_f64=orc.mse_attention_f64(q, pool, slots, B),
        attention_f32=orc.mse_attention_f32(q, pool, slots, B))
    print("wrote prod_n37_h2_d128.npz, mse_n37_h2_d128.npz")


def synthetic_records() -> None:
    import json
    sys.path.insert(0, str(HERE.parent))
    from test_synthetic import _sha, spec_inputs
    rec = {name: _sha(a) for name, a in spec_inputs().items()}
    (HERE / "synthetic_sha256.json").write_text(json.dumps(rec, indent=1) + "\n")
    print("wrote synthetic_sha256.json")


if __name__ == "__main__":
    reference_outputs()
    oracle_fixtures()
    synthetic_records()
