"""Register and LDS budgets of the persistent kernels (CPU: compiles the
kernels to gfx950 assembly and reads the code-object metadata).

The persistent kernels launch exactly as many workgroups as can be resident
at once; the encoder's cross-workgroup waits rely on it, and a workgroup that
cannot start until another exits leaves a tail.  The residency the runtime's
occupancy query reports counts VGPRs and LDS but over-estimates what the
SGPR file allows on MI355X.  Measured with a probe kernel of 256 threads,
64 VGPRs and 16.3 KiB of LDS (workgroups that start at once, of 3072):
`.amdhsa_next_free_sgpr` 72, 73, 74 -> 8 per CU; 76, 78, 80 -> 7 (the query
says 8); 96 -> 6 (the query says 7); with 80 VGPRs, 100 -> 6.  So each
kernel's SGPR count is held to what its target occupancy allows:
  * decoder: 8 waves per SIMD (64 VGPRs) and next_free_sgpr <= 74;
  * encoder: two-wave workgroups at 3 waves per SIMD (168 VGPRs, six
    workgroups per CU) and next_free_sgpr <= 100 (3 x 100 SGPRs per SIMD is
    far below the limit measured above); six workgroups' LDS must fit the
    CU's 160 KiB.
"""

from __future__ import annotations

import os
import re
import subprocess

import pytest

from conftest import PKG, REPO


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    import sys

    sys.path.insert(0, PKG)
    import build as B

    out = tmp_path_factory.mktemp("asm") / "kernels.s"
    try:
        hipcc = B.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    subprocess.run(
        [hipcc, *B.HIPCC_FLAGS, "-I", os.path.join(REPO, "include"), "-I",
         os.path.join(PKG, "csrc"), "--cuda-device-only", "-S",
         os.path.join(PKG, "csrc", "kvszp_kernels.hip"), "-o", str(out)],
        check=True, stderr=subprocess.DEVNULL)
    text = out.read_text()
    meta = {}
    for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", text, re.S):
        body = m.group(2)
        field = lambda k: int(re.search(rf"\.amdhsa_{k} (\d+)", body).group(1))
        meta[m.group(1)] = {
            "vgpr": field("next_free_vgpr"),
            "sgpr": field("next_free_sgpr"),
            "lds": field("group_segment_fixed_size"),
            "scratch": field("private_segment_fixed_size"),
        }
    # explicit (by_value) arguments of each kernel: (offset, size)
    notes = text[text.index("amdhsa.kernels:"):]
    for m in re.finditer(r"  - \.agpr_count:.*?\.args:\n(.*?)\n    \.[a-z_]+:.*?\.name:\s+(\S+)",
                         notes, re.S):
        if m.group(2) in meta:
            meta[m.group(2)]["args"] = [
                (int(o), int(z)) for o, z, kind in re.findall(
                    r"\.offset:\s+(\d+)\n\s+\.size:\s+(\d+)\n\s+\.value_kind:\s+(\S+)",
                    m.group(1)) if kind == "by_value"]
    return meta


def pick(meta, name):
    got = {k: v for k, v in meta.items() if name in k}
    assert got, f"no kernel named {name}"
    return got


def test_persistent_decoder_fits_eight_waves(kernels):
    for k, m in {**pick(kernels, "decompress_persistent_kernel"),
                 **pick(kernels, "decompress_persistent_argtable_kernel")}.items():
        assert m["vgpr"] <= 64, (k, m)
        assert m["sgpr"] <= 74, (k, m)
        assert m["lds"] <= 20480, (k, m)
        assert m["scratch"] == 0, (k, m)


def test_persistent_encoder_fits_three_waves(kernels):
    for k, m in {**pick(kernels, "compress_persistent_kernel"),
                 **pick(kernels, "compress_persistent_argtable_kernel")}.items():
        if "decompress" in k:
            continue
        assert m["vgpr"] <= 168, (k, m)
        assert m["sgpr"] <= 100, (k, m)
        assert 6 * m["lds"] <= 160 * 1024, (k, m)
        assert m["scratch"] == 0, (k, m)


def test_arg_table_layout(kernels):
    """The ArgTable launches read job records at arg_table_offset<Params>():
    the parameter block rounded up to 16 bytes (kvszp_internal.h).  The
    compiler must place the second argument exactly there, with the size
    the host copies (kArgTableBytes), and the whole argument segment must
    stay within what the runtime was measured to carry (16 648 bytes)."""
    got = {**pick(kernels, "compress_persistent_argtable_kernel"),
           **pick(kernels, "decompress_persistent_argtable_kernel")}
    assert len(got) == 7  # 4 encoder and 3 decoder instantiations
    for k, m in got.items():
        (o0, z0), (o1, z1) = m["args"]
        assert o0 == 0 and o1 == (z0 + 15) // 16 * 16, (k, m["args"])
        assert z1 == 14336, (k, m["args"])
        assert o1 + z1 <= 16648, (k, m["args"])
