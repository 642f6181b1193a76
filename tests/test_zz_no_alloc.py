"""sgemm_launch_noalloc (the entry point that allocates nothing) on the GPU.

It must give what sgemm_launch gives -- the same kernels with the same split
count, so D is bit-identical -- on two calls in a row, the second with a
smaller problem (the static scratch keeps the first call's partials and
tickets), and must reject a launch whose partials exceed the scratch before
launching anything.  Every call goes through the C-ABI (ctypes).  Captured
into a HIP graph on a caller's stream (sgemm_set_stream) -- split-K,
stream-K and edge-strip launches -- it must replay what an eager call gives.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

import oracle
from generator import catalog
from shim import sgemm_shim as S

pytestmark = pytest.mark.gpu

NAME = "mt64x64_a16_wg1x4_dk32_s3"   # carries generated_gemm_splitk; split count chosen per problem


def _say(msg):
    print(msg, flush=True)


def _kernel():
    co, toml = catalog.paths(NAME)
    return S.Kernel(co, toml)


def _problem(m, n, k, seed):
    A, B, C = S.fill_matrix(m, k, seed, 0), S.fill_matrix(k, n, seed, 1), S.fill_matrix(m, n, seed, 2)
    return A, B, C, [S.DeviceBuffer.from_array(x) for x in (A, B, C)]


def _d(kern, launch, bufs, m, n, k, alpha, beta):
    dA, dB, dC = bufs
    dD = S.DeviceBuffer(4 * m * n)
    dD.upload(np.full((m, n), np.nan, dtype=np.float32))
    getattr(kern, launch)(dA, dB, dC, dD, m, n, k, alpha=alpha, beta=beta)
    kern.synchronize()
    return dD.download().reshape(n, m).T.copy()


@pytest.mark.parametrize("first,second", [
    ((512, 512, 16384), (256, 256, 4096)),     # 4 then 16 K ranges: the second call is smaller
    ((333, 290, 5003), (70, 45, 1001)),       # ragged tiles and K remainders
])
def test_noalloc_matches_launch_on_two_calls(kernels, first, second):
    with _kernel() as ref_kern, _kernel() as kern:
        for i, (m, n, k) in enumerate((first, second)):
            splits = kern.launch_splits(m, n, k)
            _say(f"noalloc call {i + 1}: {NAME} {m}x{n}x{k}, {splits} K ranges")
            assert splits > 1, "the case must exercise the split-K scratch"
            A, B, C, bufs = _problem(m, n, k, 31 + i)
            D = _d(kern, "launch_noalloc", bufs, m, n, k, 0.5, -1.0)
            D_ref = _d(ref_kern, "launch", bufs, m, n, k, 0.5, -1.0)
            assert np.array_equal(D, D_ref), "sgemm_launch_noalloc and sgemm_launch differ"
            err = oracle.normwise_error(D, oracle.cpu_gemm_mt(A, B, C, 0.5, -1.0, threads=16))
            assert err <= oracle.tolerance(k), err


def test_noalloc_without_split_and_repeated(kernels):
    """An unsplit launch needs no workspace at all; repeated split calls on
    one device give the same bits (tickets are cleared by each call)."""
    with _kernel() as kern:
        m, n, k = 1024, 1024, 256                # 256 tiles fill the 256 CUs: no split
        _say(f"noalloc no split {m}x{n}x{k}")
        assert kern.launch_splits(m, n, k) == 1
        _, _, _, bufs = _problem(m, n, k, 41)
        assert np.array_equal(_d(kern, "launch_noalloc", bufs, m, n, k, 1.0, 1.0),
                              _d(kern, "launch", bufs, m, n, k, 1.0, 1.0))
        m, n, k = 128, 192, 8192
        _say(f"noalloc repeated {m}x{n}x{k}, {kern.launch_splits(m, n, k)} K ranges")
        _, _, _, bufs = _problem(m, n, k, 42)
        first = _d(kern, "launch_noalloc", bufs, m, n, k, 1.0, 0.0)
        for _ in range(3):
            assert np.array_equal(_d(kern, "launch_noalloc", bufs, m, n, k, 1.0, 0.0), first)


def test_noalloc_stream_k_matches_launch(kernels):
    """A stream-K launch (partials of 2 G tiles, G tickets) from the static
    scratch: the same bits as from the handle's workspace, twice in a row."""
    name = "mt128x64_a16_wg2x2_dk32_s3_occ2"
    co, toml = catalog.paths(name)
    with S.Kernel(co, toml) as ref_kern, S.Kernel(co, toml) as kern:
        groups = kern.info.stream_k_groups
        for i, (m, n, k) in enumerate(((128 * 30 - 5, 64 * 22 - 3, 333), (128 * 25, 64 * 23, 200))):
            kern.set_stream_k(2)
            ref_kern.set_stream_k(2)
            sk = kern.stream_k_tiles(m, n, k)
            _say(f"noalloc stream-K call {i + 1}: {name} {m}x{n}x{k}, {groups} groups, {sk} stream-K tiles")
            assert sk > 0 and kern.workspace_size(m, n, k) <= S.SGEMM_NOALLOC_PARTIAL_BYTES + 4 * groups
            A, B, C, bufs = _problem(m, n, k, 51 + i)
            D = _d(kern, "launch_noalloc", bufs, m, n, k, 1.0, 0.5)
            assert np.array_equal(D, _d(ref_kern, "launch", bufs, m, n, k, 1.0, 0.5))
            err = oracle.normwise_error(D, oracle.cpu_gemm_mt(A, B, C, 1.0, 0.5, threads=16))
            assert err <= oracle.tolerance(k), err


def test_noalloc_rejects_more_than_its_scratch(kernels):
    """1024^2 in 64 x 64 tiles with 16 K ranges needs 256 * 16 * 16 KiB = 64 MiB
    of partials, twice the static scratch: an error, and D is untouched."""
    with _kernel() as kern:
        kern.set_split_k(16)
        m = n = 1024
        k = 16 * 32 * 4
        need = kern.workspace_size(m, n, k)
        _say(f"noalloc oversize {m}x{n}x{k}: {need} bytes")
        assert need > S.SGEMM_NOALLOC_PARTIAL_BYTES
        _, _, _, (dA, dB, dC) = _problem(m, n, k, 43)
        dD = S.DeviceBuffer(4 * m * n)
        dD.upload(np.full((m, n), 3.0, dtype=np.float32))
        with pytest.raises(S.SgemmError, match="static scratch"):
            kern.launch_noalloc(dA, dB, dC, dD, m, n, k, alpha=1.0, beta=0.0)
        kern.synchronize()
        assert np.all(dD.download() == 3.0)


# ------------------------------------------------------------ graph capture
_vp = ctypes.c_void_p
CAPTURE_MODE_GLOBAL = 0   # hipStreamCaptureModeGlobal: any unsafe call (an allocation) fails the capture


def _ok(rc, what):
    assert rc == 0, f"{what} failed: {rc}"


GRAPH_CASES = [
    # (main, edges or None, stream-K mode or None, m, n, k): split-K, stream-K and edge-strip launches
    ("mt64x64_a16_wg1x4_dk32_s3", None, None, 256, 256, 8192),
    ("mt64x64_a16_wg1x4_dk32_s3", None, 2, 1792, 1792, 256),
    ("mt256x128_a32_wg2x2_dk16_s3_occ2", catalog.EDGE_PAIR, None, 4097, 4096, 64),
    # transposed operands: strips of the twin's own layout, and split-K on A^T
    ("mt256x128_a32_wg2x2_dk16_s3_occ2_tt", catalog.EDGE_KERNEL["mt256x128_a32_wg2x2_dk16_s3_occ2_tt"], None,
     4097, 4096, 64),
    ("mt64x64_a16_wg1x4_dk32_s3_tn", None, None, 256, 256, 8192),
]


@pytest.mark.parametrize("main,edges,mode,m,n,k", GRAPH_CASES)
def test_noalloc_launch_replays_from_a_hip_graph(kernels, main, edges, mode, m, n, k):
    _hip = ctypes.CDLL("libamdhip64.so")   # the HIP runtime the library itself links
    stream = _vp()
    _ok(_hip.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
    graph, exe = _vp(), _vp()
    opened = []
    try:
        kern = S.Kernel(*catalog.paths(main))
        opened.append(kern)
        if edges:
            strips = [S.Kernel(*catalog.paths(e)) for e in edges]
            opened += strips
            kern.set_edge_kernels(*strips)
        if mode is not None:
            kern.set_stream_k(mode)
        plan = (kern.launch_splits(m, n, k), kern.stream_k_tiles(m, n, k) if kern.info.stream_k_groups else 0,
                kern.edge_interior(m, n, k))
        _say(f"graph {main} {m}x{n}x{k}: splits, stream-K tiles, interior = {plan}")
        cfg = catalog.SOLUTIONS[main][0]
        sa = (k, m) if cfg.trans_a else (m, k)   # stored A and B
        sb = (n, k) if cfg.trans_b else (k, n)
        assert plan[0] > 1 or plan[1] > 0 or plan[2] != (m, n), "the case must use the scratch or the strips"
        dA, dB, dC, dD = S.DeviceBuffer(4 * m * k), S.DeviceBuffer(4 * k * n), S.DeviceBuffer(4 * m * n), \
            S.DeviceBuffer(4 * m * n)
        kern.set_stream(stream.value)
        # one eager call before the capture (the first call of all is captured
        # in test_first_noalloc_call_of_a_process_may_be_captured)
        dA.upload(S.fill_matrix(*sa, 1, 0))
        dB.upload(S.fill_matrix(*sb, 1, 1))
        dC.upload(S.fill_matrix(m, n, 1, 2))
        kern.launch_noalloc(dA, dB, dC, dD, m, n, k, alpha=1.5, beta=-0.5)
        kern.synchronize()
        _ok(_hip.hipStreamBeginCapture(stream, CAPTURE_MODE_GLOBAL), "hipStreamBeginCapture")
        try:
            kern.launch_noalloc(dA, dB, dC, dD, m, n, k, alpha=1.5, beta=-0.5)
        finally:
            _ok(_hip.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
        _ok(_hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
        for replay in range(3):
            seed = 50 + replay
            A, B, C = S.fill_matrix(*sa, seed, 0), S.fill_matrix(*sb, seed, 1), S.fill_matrix(m, n, seed, 2)
            dA.upload(A)
            dB.upload(B)
            dC.upload(C)
            dD.upload(np.full((m, n), np.nan, dtype=np.float32))
            _ok(_hip.hipGraphLaunch(exe, stream), "hipGraphLaunch")
            _ok(_hip.hipStreamSynchronize(stream), "hipStreamSynchronize")
            D_graph = dD.download().reshape(n, m).T.copy()
            dD.upload(np.full((m, n), np.nan, dtype=np.float32))
            kern.launch_noalloc(dA, dB, dC, dD, m, n, k, alpha=1.5, beta=-0.5)
            kern.synchronize()
            D_eager = dD.download().reshape(n, m).T.copy()
            _say(f"  replay {replay}: checking")
            assert np.array_equal(D_graph, D_eager), f"replay {replay} differs from the eager launch"
            opA = np.asfortranarray(A.T) if cfg.trans_a else A
            opB = np.asfortranarray(B.T) if cfg.trans_b else B
            err = oracle.normwise_error(D_graph, oracle.cpu_gemm_mt(opA, opB, C, 1.5, -0.5, threads=16))
            assert err <= oracle.tolerance(k), (replay, err)
    finally:
        if exe.value:
            _hip.hipGraphExecDestroy(exe)
        if graph.value:
            _hip.hipGraphDestroy(graph)
        for kk in opened:
            kk.set_stream(None)
        for kk in reversed(opened):
            kk.close()
        _hip.hipStreamDestroy(stream)


FIRST_CAPTURE_CHILD = r"""
import ctypes, sys
import numpy as np
sys.path[:0] = sys.argv[1:4]
import oracle
from generator import catalog
from shim import sgemm_shim as S
hip = ctypes.CDLL("libamdhip64.so")
vp = ctypes.c_void_p
def ok(rc, what):
    assert rc == 0, f"{what} failed: {rc}"
name, (m, n, k) = "mt64x64_a16_wg1x4_dk32_s3", (256, 256, 8192)
kern = S.Kernel(*catalog.paths(name))
ref = S.Kernel(*catalog.paths(name))
assert kern.launch_splits(m, n, k) > 1
stream, graph, exe = vp(), vp(), vp()
ok(hip.hipStreamCreate(ctypes.byref(stream)), "hipStreamCreate")
A, B, C = S.fill_matrix(m, k, 7, 0), S.fill_matrix(k, n, 7, 1), S.fill_matrix(m, n, 7, 2)
dA, dB, dC = (S.DeviceBuffer.from_array(x) for x in (A, B, C))
dD, dR = S.DeviceBuffer.from_array(np.full((m, n), np.nan, np.float32)), S.DeviceBuffer(4 * m * n)
kern.set_stream(stream.value)
print("capturing the first sgemm_launch_noalloc of this process", flush=True)
ok(hip.hipStreamBeginCapture(stream, 0), "hipStreamBeginCapture")
try:
    kern.launch_noalloc(dA, dB, dC, dD, m, n, k, alpha=1.5, beta=-0.5)
finally:
    ok(hip.hipStreamEndCapture(stream, ctypes.byref(graph)), "hipStreamEndCapture")
ok(hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
ref.launch(dA, dB, dC, dR, m, n, k, alpha=1.5, beta=-0.5)
ref.synchronize()
R = dR.download().reshape(n, m).T.copy()
for replay in range(3):
    dD.upload(np.full((m, n), np.nan, np.float32))
    ok(hip.hipGraphLaunch(exe, stream), "hipGraphLaunch")
    ok(hip.hipStreamSynchronize(stream), "hipStreamSynchronize")
    D = dD.download().reshape(n, m).T.copy()
    assert np.array_equal(D, R), f"replay {replay} differs from sgemm_launch"
    err = oracle.normwise_error(D, oracle.cpu_gemm_blocked(A, B, C, 1.5, -0.5, threads=8))
    assert err <= oracle.tolerance(k), err
    print(f"replay {replay}: equal to sgemm_launch, normwise error {err:.3e}", flush=True)
hip.hipGraphExecDestroy(exe)
hip.hipGraphDestroy(graph)
kern.set_stream(None)
kern.close()
ref.close()
hip.hipStreamDestroy(stream)
print("FIRST_CAPTURE_OK", flush=True)
"""


def test_first_noalloc_call_of_a_process_may_be_captured(kernels):
    """sgemm_open looks up the static scratch's device address, so the very
    first sgemm_launch_noalloc of a process (split-K, using the scratch) may
    run under graph capture: in a fresh child process, capture it first,
    replay the graph three times and compare each replay with sgemm_launch."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    paths = [os.path.join(root, "amdgpu-arch-gemm_amd"), os.path.join(root, "oracle"), root]
    _say("child process: first no-alloc call under capture")
    ret = subprocess.run([sys.executable, "-u", "-c", FIRST_CAPTURE_CHILD] + paths, stdout=subprocess.PIPE,
                         stderr=subprocess.STDOUT, timeout=300)
    out = ret.stdout.decode()
    _say(out)
    assert ret.returncode == 0 and "FIRST_CAPTURE_OK" in out, out

