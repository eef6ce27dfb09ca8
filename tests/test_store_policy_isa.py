"""The output store policy survives compilation.

Every forward kernel is built twice, KEEP=false (outputs streamed with
non-temporal stores, the fast form for an op whose result is not read next)
and KEEP=true (plain stores that leave the output in L2 / the Infinity Cache
for the next op of a chain).  Results are the same bits either way, so no
numeric test can see a lost hint; this one compiles the kernel sources to
gfx950 assembly and checks every 16-byte global store: `nt` (alone, or with
the write-through scope `sc1`) in the streamed variants, plain in the kept
ones (add+RMSNorm's residual output is a plain store in both, measured the
faster form beside the streamed y).  The backward
kernels and the device copy take the same parameter; the LayerNorm
backward's dgamma/dbeta slot partials (ln_bwd_vec, and lr_bwd_apply over
long rows, which also adds into dgamma / dbeta in place) are plain stores
in both variants (the slot sums read them back next).  The runtime's fused
kernels (fused_chain_vec, and the LayerNorm with an epilogue) stream the
intermediates a later layer reads and store only the group's last output
by KEEP: the kept variant has both kinds of store, the streamed one only
non-temporal stores."""
import os
import re
import shutil
import subprocess

import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "mimir-framework_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fno-gpu-flush-denormals-to-zero", "-Xclang",
         "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S"]
SOURCES = ["elementwise", "norm", "softmax", "gather", "rope", "longrow", "backward", "runtime"]
# Kernels of backward.hip / runtime.hip whose last template parameter is KEEP.
KEEP_KERNELS = ("dact_vec", "mul_bwd_vec", "add_bwd_vec", "acc_vec", "ln_bwd_vec", "copy16_kernel")


def _stores_by_kernel(asm):
    stores, name = {}, None
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            name = m.group(1)
            stores[name] = []
            continue
        code = line.split(";")[0]
        if name and "global_store_dwordx4" in code:
            stores[name].append(bool(re.search(r"\bnt\b", code)))
    return stores


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", SOURCES)
def test_keep_variants_store_as_intended(src, tmp_path):
    out = tmp_path / f"{src}.s"
    r = subprocess.run([HIPCC, *FLAGS, "-o", str(out), os.path.join(CSRC, f"{src}.hip")],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    checked = 0
    for name, nt in _stores_by_kernel(out.read_text()).items():
        if not nt:
            continue
        norm = re.search(r"norm_rows_vec\S*Lb([01])ELb([01])ELb[01]EEEv", name)  # <..., KEEP, EPI, FULL>
        chain = re.search(r"fused_chain_vecILb([01])E", name)
        if (norm and norm.group(2) == "1") or chain:  # intermediates streamed; the last output by KEEP
            checked += 1
            if (norm or chain).group(1) == "1":
                assert any(nt) and not all(nt), f"{name}: {nt}"
            else:
                assert all(nt), f"{name}: a streamed output lost its non-temporal hint"
            continue
        # KEEP is the last template parameter, or the one before the trailing
        # workgroup shape (the streaming kernels' BS, the long-row apply
        # pass's BS and VPT).
        tail = re.search(r"Lb([01])E(?:Li\d+E)*EEv", name)
        keep = norm.group(1) == "1" if norm else bool(tail and tail.group(1) == "1")
        if not (norm or tail):
            continue  # not a KEEP-templated kernel
        if src in ("backward", "runtime") and not any(k in name for k in KEEP_KERNELS):
            continue  # a bool template parameter that is not KEEP
        checked += 1
        if not keep and "NormE2E" in name:  # add+RMSNorm: r_out plain, y streamed
            assert nt.count(True) == nt.count(False), f"{name}: {nt}"
        elif ("ln_bwd_vec" in name or "lr_bwd_apply" in name) and not keep:  # dx streamed, slot partials plain
            assert any(nt), f"{name}: dx lost its non-temporal hint"
        elif keep:
            assert not any(nt), f"{name}: a kept output is stored non-temporal"
        else:
            assert all(nt), f"{name}: a streamed output lost its non-temporal hint"
    assert checked >= 2, f"{src}: no KEEP variants found"
