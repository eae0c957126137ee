"""LGX_TRACE, the env-gated launch trace (after LOGOS_TIER_TRACE,
crates/logicaffeine_compile/src/vm/tier_trace.rs:1-29): set, non-empty and not
"0", it writes one stderr line per kernel launch, binary16 GEMM call and graph
replay; otherwise nothing.  The library reads the variable once per process,
so each case runs in a child process of its own (one GEMV, a tiny model's
prefill in both modes, and graph-replayed decode steps).
"""
import os
import re
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CHILD = r"""
import sys
import numpy as np
import logicaffeine_amd as lgx
from oracle import oracle as orc

ctx = lgx.Context(0)
rng = np.random.default_rng(5)
n, k = 256, 512
qs = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
d = orc.f32_to_f16(np.full((n, k // 32), 0.01, np.float32))
W = ctx.q8_matrix(qs, d)
y = ctx.q8_gemv_f32(W, ctx.to_device(rng.standard_normal(k).astype(np.float32)))
y.cpu()
print("gemv launches", ctx.launch_count, flush=True)
cfg = orc.qwen_config("tiny")
m = lgx.Model(ctx, cfg, 3)
prompt = ctx.to_device(rng.integers(0, cfg["vocab"], size=(2, 12)).astype(np.int32))
tok = m.prefill(prompt)
m.generate(tok, 3)
m.reset()
m.set_prefill_mode(True)
tok = m.prefill(prompt)
tok.cpu()
print("done launches", ctx.launch_count, flush=True)
m.close()
ctx.close()
"""


def _run(value):
    env = dict(os.environ)
    env.pop("LGX_TRACE", None)
    if value is not None:
        env["LGX_TRACE"] = value
    print(f"[trace] child with LGX_TRACE={value!r}", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD], cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    return r.stdout, [ln for ln in r.stderr.splitlines() if ln.startswith("[lgx] ")]


def _launches(stdout, tag):
    return int(re.search(rf"^{tag} launches (\d+)$", stdout, re.M).group(1))


def test_trace_lines_one_per_launch():
    out, lines = _run("1")
    launch = [ln for ln in lines if ln.startswith("[lgx] launch ")]
    pat = re.compile(r"^\[lgx\] launch dev=0 n=(\d+) (lgx_k_\w+) grid=(\d+)x(\d+)x(\d+) "
                     r"block=(\d+)x(\d+)x(\d+) lds=\d+ stream=\S+( captured)?$")
    assert all(pat.match(ln) for ln in launch), [ln for ln in launch if not pat.match(ln)][:5]
    # one line per counted launch, numbered in order
    ns = [int(pat.match(ln).group(1)) for ln in launch]
    assert ns == list(range(_launches(out, "done")))
    first = launch[:_launches(out, "gemv")]
    assert any(" lgx_k_q8_gemv" in ln for ln in first), first
    for ln in launch:
        g = [int(v) for v in pat.match(ln).groups()[2:8]]
        assert min(g) >= 1 and g[3] * g[4] * g[5] <= 1024, ln
    # the decode step recorded into a graph once, then three replays
    assert any(ln.endswith(" captured") for ln in launch)
    replays = [ln for ln in lines if ln.startswith("[lgx] graph ")]
    assert [re.search(r"step=(\d+)", ln).group(1) for ln in replays] == ["0", "1", "2"], replays
    assert all(" replay B=2 " in ln for ln in replays)
    # the fast prefill's binary16 GEMMs
    gemm = [ln for ln in lines if ln.startswith("[lgx] gemm ")]
    assert gemm and all(re.match(r"^\[lgx\] gemm dev=0 hipblaslt m=\d+ n=\d+ k=\d+ out=f(16|32) stream=\S+$",
                                 ln) for ln in gemm), gemm[:5]
    assert any("out=f16" in ln for ln in gemm) and any("out=f32" in ln for ln in gemm)


@pytest.mark.parametrize("value", [None, "", "0"])
def test_trace_off(value):
    out, lines = _run(value)
    assert _launches(out, "done") > 0
    assert lines == []
