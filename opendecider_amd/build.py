"""Builds the gfx950 HIP library `libod_mi355x.so` in-tree with hipcc.

    python -m opendecider_amd.build            # compile every kernel source and link the shared library

Each source is compiled to an object in parallel under opendecider_amd/_build/, then linked. Flags:
  --offload-arch=gfx950                the only target (MI355X)
  -ffp-contract=off                    no implicit FMA contraction: the quantizer and the GEMM epilogue are held to
                                       a fixed fp32 operation order (kernels write fmaf where they want one)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                                       no packed fp32 instructions (v_pk_{add,mul,fma}_f32) anywhere
fp32 division stays IEEE correctly rounded (hipcc's default); the quantizer depends on it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libod_mi355x.so")
SOURCES = ["od_quant.hip", "od_gemm.hip", "od_attn.hip", "od_wide.hip", "od_layer.hip", "od_lmhead.hip", "od_gdn.hip",
           "od_gdn_chunk.hip"]
# the matrix-core ceiling probe bench.py reports beside the rooflines, in a library of its own
PROBE_SOURCE = "od_probe.hip"
PROBE_LIB = os.path.join(PKG, "libod_probe.so")
# per-source flags: the chunked GDN kernel feeds its MFMA accumulators to vector ALU work every step, so they are
# kept in ordinary VGPRs (no accumulator-register copies); so do the attention kernels (softmax and rescale on the
# score and output accumulators): at head_dim 256 (one wave per SIMD, 512 registers) the accumulator-register form
# moved them between register files every block and spilled to scratch, the VGPR form does neither (the staged
# path 0.92x and the int8 path 0.79x the time, bit-identical; the wide attention's LDS-DMA kernel at head_dim 256
# fits 220 VGPRs and two workgroups per CU with it); at head_dims 64 / 128 no accumulator register is used either way
SOURCE_FLAGS = {"od_gdn_chunk.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "od_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
                "od_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-inline-asm"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; that line is expected
    out = "\n".join(ln for ln in r.stdout.splitlines() if "packed-fp32-ops" not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    return out


def build(verbose: bool = False) -> str:
    """Compile every kernel source for gfx950 and link libod_mi355x.so (and libod_probe.so). Returns the path of
    libod_mi355x.so."""
    os.makedirs(BUILD, exist_ok=True)
    objs = [os.path.join(BUILD, s.replace(".hip", ".o")) for s in SOURCES]
    cmds = [[HIPCC, *FLAGS, *SOURCE_FLAGS.get(s, []), "-c", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(SOURCES, objs)]
    probe_obj = os.path.join(BUILD, PROBE_SOURCE.replace(".hip", ".o"))
    cmds.append([HIPCC, *FLAGS, "-c", os.path.join(CSRC, PROBE_SOURCE), "-o", probe_obj])
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        outs = list(ex.map(_run, cmds))
    for lib, lib_objs in ((LIB, objs), (PROBE_LIB, [probe_obj])):
        tmp = lib + ".tmp"
        outs.append(_run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *lib_objs, "-o", tmp]))
        os.replace(tmp, lib)
    if verbose:
        for o in outs:
            if o.strip():
                print(o)
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
