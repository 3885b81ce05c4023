"""CPU check of the hot kernels' register budgets, from the compiler's own resource report
(hipcc -Rpass-analysis=kernel-resource-usage on the device pass, the library's build flags).

Each kernel's speed rests on a register budget stated in its source: two waves per SIMD for
the prefill forward, the dK/dV producer/consumer pair and the dQ-from-dS kernel (at most 256
registers a lane, AGPRs included), and no scratch in any hot kernel (a spill puts memory
round trips into the inner loop).  A source change that pushes one past its budget still
compiles and still passes every parity test, only slower; this test names it instead.
No GPU is used."""
import os
import re
import shutil
import subprocess

import pytest

from transformer_amd import build as B

HOT = {
    # file: [(kernel name regex, max VGPR + AGPR per lane)]
    "prefill_fwd.hip": [(r"prefill_fwd_kernelILi128ELi1ELb0ELb0E", 256), (r"prefill_fwd_kernelILi128ELi1ELb0ELb1E", 256)],
    "prefill_bwd.hip": [(r"bwd_dkdv_kernelILi128E", 256), (r"bwd_dq_ds_kernelILi128E", 256)],
    "decode.hip": [(r"decode_kernelILi512ELb1E", 512), (r"decode_merge_uv_kernelILi512E", 256)],
    "prefill_cached.hip": [(r"prefill_cached_kernelILi512ELi8E", 256), (r"prefill_cached_kernelILi512ELi4E", 256)],
    "linear_rows.hip": [(r"linear_rows_kernelILi1E", 256), (r"linear_rows_kernelILi2E", 256),
                        (r"linear_rows_rope_append_kernelILi1E", 256), (r"linear_rows_rope_append_kernelILi2E", 256)],
}


def resources(src: str) -> dict:
    """{mangled kernel name: {"VGPRs": n, "AGPRs": n, "ScratchSize": bytes}} from the compiler."""
    name = os.path.basename(src)
    cmd = [B.HIPCC, *B.FLAGS, *B.FILE_FLAGS.get(name, []), "-I", B.CSRC, "--offload-device-only",
           "-Rpass-analysis=kernel-resource-usage", "-c", src, "-o", os.devnull]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out, cur = {}, None
    for line in r.stderr.splitlines():
        m = re.search(r"remark:\s+(Function Name|VGPRs|AGPRs|ScratchSize \[bytes/lane\]): (\S+)", line)
        if not m:
            continue
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = out.setdefault(val, {})
        elif cur is not None:
            cur[key.split(" ")[0]] = int(val)
    return out


@pytest.mark.skipif(not shutil.which(B.HIPCC) and not os.path.exists(B.HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", sorted(HOT))
def test_hot_kernels_fit_their_register_budgets(src):
    res = resources(os.path.join(B.CSRC, src))
    for pattern, max_regs in HOT[src]:
        found = [k for k in res if re.search(pattern, k)]
        assert found, f"{src}: no kernel matches {pattern}"
        for k in found:
            r = res[k]
            assert {"VGPRs", "AGPRs", "ScratchSize"} <= set(r), f"{k}: incomplete resource report {r}"
            regs = r["VGPRs"] + r["AGPRs"]
            assert r["ScratchSize"] == 0, f"{k} spills {r['ScratchSize']} bytes per lane"
            assert regs <= max_regs, f"{k} uses {regs} registers per lane, budget {max_regs}"
