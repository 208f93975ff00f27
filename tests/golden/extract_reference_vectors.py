#!/usr/bin/env python3
"""Collect the reference's recorded oracle vectors into a small JSON fixture.

Reads the reference's result files (data, not source) under
``/root/reference/bench/results/m0`` and writes ``reference_vectors.json``
next to this script.  Only the fields that pin arithmetic are kept: the
probe parameters, the CPU-oracle checksum, the first eight oracle outputs,
and the SHA-256 of the datasets the reference wrote.  Run it in a container
that has the reference mounted; the GPU tests never need it.
"""

from __future__ import annotations

import json
from pathlib import Path

RESULTS = Path("/root/reference/bench/results/m0")
OUT = Path(__file__).with_name("reference_vectors.json")

QMV_FILES = [
    "native-m1-top8-gather-simdmap-gate-up-qmv-q8.json",
    "native-m1-top8-gather-simdmap-gate-up-qmv-q4.json",
    "native-m1-top8-gather-simdmap-down-qmv-q8.json",
    "native-m1-top8-gather-simdmap-down-qmv-q4.json",
    "native-m1-top8-contiguous-bank-gate-up-qmv-q8.json",
    "native-m1-top8-contiguous-bank-gate-up-qmv-q4.json",
    "native-m1-top8-gate-up-qmv-q8.json",
    "native-m1-top8-gate-up-qmv-q4.json",
    "native-m1-top8-down-qmv-q8.json",
    "native-m1-top8-down-qmv-q4.json",
    "native-m1-ornith-shape-weight-major-qmv-q8.json",
    "native-m1-ornith-shape-weight-major-qmv-q4.json",
    "native-m1-weight-major-qmv-q8.json",
    "native-m1-weight-major-qmv-q4.json",
]
FUSED_FILES = [
    "native-m1-two-stage-moe-q8-512.json",
    "native-m1-two-stage-moe-q4-512.json",
    "native-m1-two-stage-moe-q8-256.json",
    "native-m1-two-stage-moe-q4-256.json",
    "native-m1-fused-moe-q8.json",
    "native-m1-fused-moe-q4.json",
]
QMM_FILES = [
    "native-m1-qmm-4d-q8-m64-n4096-k2048-r256.json",
    "native-m1-qmm-4d-q4-m64-n4096-k2048-r256.json",
]
MLX_FILES = [
    "mlx-current-ornith-shape-qmv-q8.json",
    "mlx-current-ornith-shape-qmv-q4.json",
]


def main() -> int:
    out: dict[str, list] = {"qmv": [], "fused": [], "qmm": [], "mlx_qmv": []}
    for name in QMV_FILES:
        d = json.loads((RESULTS / name).read_text())
        p = d["protocol"]
        m = d["measurements"][0]
        out["qmv"].append({
            "source": f"bench/results/m0/{name}",
            "bits": 4 if p["bits"] == "q4" else 8,
            "output_size": p["output_size"],
            "reduction_size": p["reduction_size"],
            "group": p["quant_group_size"],
            "bank_rows": p.get("weight_bank_output_size", 0),
            "rows_per_expert": p.get("rows_per_expert", 0),
            "selected": p.get("selected_experts", []),
            "reference_checksum": m["reference_checksum"],
            "first_reference": m["first_reference"],
        })
    for name in FUSED_FILES:
        d = json.loads((RESULTS / name).read_text())
        p = d["protocol"]
        m = d["measurements"][0]
        out["fused"].append({
            "source": f"bench/results/m0/{name}",
            "bits": 4 if p["bits"] == "q4" else 8,
            "total_experts": p["total_experts"],
            "selected": p["selected_experts"],
            "schedule": p["schedule"],
            "reference_checksum": m["reference_checksum"],
            "recorded_gpu_output_checksum": m["output_checksum"],
        })
    for name in QMM_FILES:
        d = json.loads((RESULTS / name).read_text())
        p = d["protocol"]
        m = d["measurement"]
        out["qmm"].append({
            "source": f"bench/results/m0/{name}",
            "bits": 4 if p["bits"] == "q4" else 8,
            "tokens": p["tokens"],
            "outputs": p["outputs"],
            "reduction_size": p["reduction_size"],
            "reference_checksum": m["reference_checksum"],
        })
    for name in MLX_FILES:
        d = json.loads((RESULTS / name).read_text())
        p = d["protocol"]
        c = d["correctness"]
        out["mlx_qmv"].append({
            "source": f"bench/results/m0/{name}",
            "bits": p["bits"],
            "output_size": p["output_size"],
            "reduction_size": p["reduction_size"],
            "group": p["group_size"],
            "dataset_sha256": p["dataset_sha256"],
            "mlx_output_checksum": c["output_checksum"],
            "numpy_reference_checksum": c["reference_checksum"],
            "max_absolute_error": c["max_absolute_error"],
        })
    OUT.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
