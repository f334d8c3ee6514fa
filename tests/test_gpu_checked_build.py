"""The device bounds-check build (libssalaad_amd_checked.so, SSL_DEVICE_CHECKS=1).

Run in a child process, so that its library and status words stay apart from
this process's:
  * valid calls on the streaming, split-row, prefill (parts included), chained
    and in-place paths record nothing and match the oracle;
  * a negative column index written into a module's device structure after
    planning is clamped and recorded (status word bit 9), and the call ends
    normally; the same for the in-place op (the library's own word);
  * an out-of-range block-row written into a prefill group record is dropped
    and recorded (bit 10).
The child first asserts that it loaded the checked build: only its kernels
turn those indices into a record instead of an access.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
CHECKED = ROOT / "s-salaad_amd" / "ssalaad_amd" / "libssalaad_amd_checked.so"

pytestmark = pytest.mark.gpu

CHILD = r'''
import ctypes, json, sys
from pathlib import Path
sys.path[:0] = [ROOT, ROOT + "/s-salaad_amd", ROOT + "/tests"]
import numpy as np, torch
from slr_cases import TOL, err, make_module, make_problem, make_x, oracle_y, to_dev
from oracle import slr_oracle as orc
from ssalaad_amd import _lib, _runtime, LRSLinearChain
import ssalaad_amd
lib = _lib.load()
assert lib.ssl_device_checks() == 1, "not the checked build"
dev = torch.device("cuda:0")
hip = ctypes.CDLL(str(Path(torch.__file__).parent / "lib" / "libamdhip64.so"))
def poke(t, index, value):
    """Write one int32 into device memory behind torch's back (no version bump)."""
    v = ctypes.c_int32(value)
    assert hip.hipMemcpy(ctypes.c_void_p(t.data_ptr() + 4 * index), ctypes.byref(v), 4, 1) == 0
out = {}
bf = torch.bfloat16
status = lambda: (torch.cuda.synchronize(), _runtime.status_word(dev).read())[1]
# valid calls: streaming, split rows, prefill with parts, chain, op
prob = make_problem(512, 1024, 64, 32, 0.5, bf, seed=1)
mod = make_module(prob, dev)
errs = []
for M in (1, 16, 300):
    x = make_x(prob, M, seed=M)
    errs.append(err(mod(to_dev(x, bf, dev)), oracle_y(prob, x)))
skew = make_problem(4096, 8192, 64, 64, 0.1, bf, seed=2, skew=True)
ms = make_module(skew, dev)
xs = make_x(skew, 2048, seed=3)
errs.append(err(ms(to_dev(xs, bf, dev)), oracle_y(skew, xs)))
nxt = make_module(make_problem(256, 512, 64, 32, 0.5, bf, seed=4), dev)
ch = LRSLinearChain([[mod], [nxt]], [mod])
ch(to_dev(make_x(prob, 8), bf, dev))
crow32, col32, vt, act = orc.module_buffers(prob["crow"], prob["col"], prob["vals"])
o = torch.zeros(40, 512, dtype=bf, device=dev)
for M in (40,):
    torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(
        o, to_dev(make_x(prob, M), bf, dev), torch.from_numpy(crow32).to(dev),
        torch.from_numpy(col32).to(dev), to_dev(vt, bf, dev), torch.from_numpy(act).to(dev))
out["valid_err"] = max(errs)
out["valid_status"] = status()
out["valid_op_word"] = lib.ssl_debug_check_word()
# a bad column index in the module's device structure (the plan is already built)
st = mod._kernel()
poke(st.col, 3, -7)
mod(to_dev(make_x(prob, 16), bf, dev))
out["column_status"] = status()
ssalaad_amd.clear_wait_status(dev)
# the op: a bad column in its device column array
col_dev = torch.from_numpy(col32).to(dev)
args = (to_dev(make_x(prob, 40), bf, dev), torch.from_numpy(crow32).to(dev), col_dev,
        to_dev(vt, bf, dev), torch.from_numpy(act).to(dev))
torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(o, *args)   # plans from the good copy
poke(col_dev, 0, -5)
torch.ops.ssalaad.tilelang_bsr_addmm_inplace_dense_(o, *args)
torch.cuda.synchronize()
out["op_word"] = lib.ssl_debug_check_word()
# a bad block-row in a prefill group record
p2 = make_problem(1024, 1024, 64, 64, 0.5, bf, seed=5)
m2 = make_module(p2, dev)
x2 = to_dev(make_x(p2, 512), bf, dev)
m2(x2)
s2 = m2._kernel()
G = int(lib.ssl_prefill_group(512, s2.NB, 64, 64))
poke(s2.prefill_plan(G).groups, 2, 1 << 20)   # group 0's first block-row
m2(x2)
out["group_status"] = status()
ssalaad_amd.clear_wait_status(dev)
print("RESULT " + json.dumps(out), flush=True)
'''


def test_checked_build_records_nothing_on_valid_calls_and_catches_bad_indices(gpu_device):
    assert CHECKED.exists(), "build the checked variant: python s-salaad_amd/build.py --checked"
    env = dict(os.environ, SSALAAD_AMD_LIB=str(CHECKED))
    code = "ROOT = " + repr(str(ROOT)) + "\n" + CHILD
    print("[checked] child process with the checked build", flush=True)
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=240)
    assert res.returncode == 0, res.stderr[-3000:]
    line = [ln for ln in res.stdout.splitlines() if ln.startswith("RESULT ")][-1]
    out = json.loads(line[len("RESULT "):])
    assert out["valid_err"] <= 1e-2
    assert out["valid_status"] == 0 and out["valid_op_word"] == 0
    assert out["column_status"] == 1 << (8 + 1)
    assert out["op_word"] == 1 << (8 + 1)
    assert out["group_status"] == 1 << (8 + 2)
