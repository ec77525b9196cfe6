"""Static checks of the gfx950 code objects built into the library's objects
(fluidaudio-web_amd/csrc/_build/*.o), read from each kernel's AMDGPU metadata
note: the kernels of the encoder, log-mel, decoder and streaming paths use no
scratch memory and spill no registers, fit their LDS in the CU's 160 KB, and
name a workgroup size the launches respect (checked per launch by the launch
audit).  CPU only."""
from __future__ import annotations

import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BUILD = os.path.join(os.path.dirname(HERE), "fluidaudio-web_amd", "csrc", "_build")
sys.path.insert(0, os.path.join(HERE, "audit"))

# kernel name fragments of the hot paths (mangled names)
PATH_KERNELS = ("gemm_dma_kernel", "gemm_skinny", "gemm_f32_kernel", "relpos_attn_t_kernel", "stream_attn_kernel", "enc_ln", "sub_c01_kernel",
                "sub_dw_kernel", "dwconv_", "mel_frames_kernel", "mel_stats_kernel", "mel_norm_kernel", "tdt_", "stream_", "wdq_kernel",
                "copy_f4_kernel", "set_mel_src_kernel", "gemv_batch_kernel")


def _kernels():
    msgpack = pytest.importorskip("msgpack")  # noqa: F841 (build_audit reads the notes with it)
    import build_audit as b
    if not os.path.isdir(BUILD) or not any(f.endswith(".o") for f in os.listdir(BUILD)):
        pytest.skip("library objects not built (run __graft_entry__.build())")
    out = {}
    for f in sorted(os.listdir(BUILD)):
        if not f.endswith(".o"):
            continue
        blob = open(os.path.join(BUILD, f), "rb").read()
        for co in b._code_objects(blob):
            for k in b._metadata(co).get("amdhsa.kernels", []):
                out[k[".name"]] = k
    return out


def test_path_kernels_use_no_scratch_and_spill_nothing():
    ks = _kernels()
    path = {n: k for n, k in ks.items() if any(p in n for p in PATH_KERNELS)}
    assert len(path) > 50, len(path)
    bad = [(n, k.get(".sgpr_spill_count", 0), k.get(".vgpr_spill_count", 0), k.get(".private_segment_fixed_size", 0)) for n, k in path.items()
           if k.get(".sgpr_spill_count", 0) or k.get(".vgpr_spill_count", 0) or k.get(".private_segment_fixed_size", 0)]
    assert bad == [], bad


def test_every_kernel_fits_lds_and_names_its_workgroup_bound():
    for n, k in _kernels().items():
        assert k.get(".group_segment_fixed_size", 0) <= 160 * 1024, n
        assert 0 < k.get(".max_flat_workgroup_size", 1024) <= 1024, n
