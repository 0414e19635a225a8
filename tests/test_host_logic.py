"""CPU checks of host-side logic that needs no GPU."""
import pytest


def test_kernel_ready_copies_overlapping_rows():
    """A broadcast view (row stride 0) must not reach a kernel as a matrix
    with ld = #columns: _kernel_ready copies it, and _ld refuses it."""
    import torch
    from nlearn_amd.kernels.gemm import _kernel_ready, _ld

    b = torch.ones(8, dtype=torch.bfloat16).expand(4, 8)
    assert b.stride() == (0, 1)
    with pytest.raises(ValueError, match="overlap"):
        _ld(b)
    r = _kernel_ready(b)
    assert r.shape == (4, 8) and r.stride(0) >= 8 and torch.equal(r, b)
    # a dense or padded matrix is passed through untouched
    d = torch.zeros((4, 16), dtype=torch.bfloat16)[:, :12]
    assert _kernel_ready(d).data_ptr() == d.data_ptr() and _ld(d) == 16
    one = torch.zeros((1, 12), dtype=torch.bfloat16)
    assert _ld(one) == 16


def test_padded_empty_row_strides():
    """Rows start on 16-byte boundaries; rows of 1024 columns or more on
    128-byte lines, and a stride that is a multiple of 1024 elements gets 64 more."""
    import torch
    from nlearn_amd.kernels.gemm import padded_empty

    cases = {(3, 12): 16, (3, 512): 512, (3, 1000): 1000, (3, 1536): 1536, (3, 2048): 2112, (3, 4096): 4160,
             (3, 2040): 2112, (3, 50257): 50304}
    for (r, c), ld in cases.items():
        t = padded_empty(r, c, torch.bfloat16, "cpu")
        assert t.shape == (r, c) and t.stride() == (ld, 1), (c, t.stride())


def _bench_module():
    import importlib.util
    import os

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench.py")
    spec = importlib.util.spec_from_file_location("nlearn_bench", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod, path


def test_bench_refuses_more_than_one_gpu():
    """The bench measures one GPU: --gpus above 1 exits with status 2 and says so."""
    import subprocess
    import sys

    _, path = _bench_module()
    r = subprocess.run([sys.executable, path, "--gpus", "2"], capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_bench_variant_failure_is_reported_not_raised(monkeypatch):
    """A failure of the bs4 x seq4096 variant ends up in its detail entry, so
    the headline JSON line is still printed."""
    mod, _ = _bench_module()

    def boom(*args, **kwargs):
        raise RuntimeError("HIP out of memory")

    monkeypatch.setattr(mod, "run_workload", boom)
    got = mod.variant_detail(None, None, 50, 10, True, None)
    assert got == {"error": "RuntimeError: HIP out of memory"}


def test_busy_stats_counts_overlap_once():
    """The busy ratio is the union of kernel intervals over the replay window
    (from the first of the last `steps` step starts, marked by the embedding
    kernel, to the last kernel's end). Per step here: the embedding [0, 100),
    A [100, 500) and B [300, 700) overlapping by 200, C [800, 900): union 800
    of a 1000 ns step, kernel sum 1000. A warm-up step before the window is
    left out."""
    bench, _ = _bench_module()
    rows = []
    for t in (0, 1000, 2000, 3000):
        rows += [(t, t + 100, "void nl::(anonymous namespace)::embed_fwd_kernel(int, int)"),
                 (t + 100, t + 500, "void nl::(anonymous namespace)::gemm2_kernel<128, 128>(nl::GemmArgs)"),
                 (t + 300, t + 700, "void nl::(anonymous namespace)::ln_bwd_kernel<1>(int)"),
                 (t + 800, t + 900, "void nl::(anonymous namespace)::mean_kernel(float const*, int, float*)")]
    out = bench.busy_stats(rows, steps=3, bs=2, seq=8)
    wall = 3900 - 1000
    assert out["replays"] == 3
    assert out["busy_ratio"] == round(3 * 800 / wall, 4)
    assert out["kernel_sum_over_wall"] == round(3 * 1000 / wall, 4)
    assert out["wall_ms_per_step"] == round(wall / 3 / 1e6, 4)
    k = out["kernels_ms_per_step"]
    assert set(k) == {"embed_fwd_kernel", "gemm2_kernel<128, 128>", "ln_bwd_kernel<1>", "mean_kernel"}
    assert k["gemm2_kernel<128, 128>"] == {"ms": round(400 / 1e6, 4), "calls": 1.0}
    with pytest.raises(SystemExit):
        bench.busy_stats(rows, steps=4, bs=2, seq=8)   # needs one step start more than the window holds


def test_train_step_refuses_fewer_hardware_queues_than_tested(monkeypatch):
    """GPU_MAX_HW_QUEUES below 4 (a 2-queue process once ended in a host
    segmentation fault of unknown cause) is refused when the step is built,
    before anything touches the GPU; 4 and more, unset or unparsable pass."""
    from nlearn_amd import train as tr

    for bad in ("1", "2", "3"):
        with pytest.raises(RuntimeError, match="GPU_MAX_HW_QUEUES"):
            tr.check_hw_queues({"GPU_MAX_HW_QUEUES": bad})
    for ok in ({}, {"GPU_MAX_HW_QUEUES": "4"}, {"GPU_MAX_HW_QUEUES": "16"}, {"GPU_MAX_HW_QUEUES": "x"}):
        tr.check_hw_queues(ok)
    monkeypatch.setenv("GPU_MAX_HW_QUEUES", "2")
    with pytest.raises(RuntimeError, match="at least 4"):
        tr.make_train_step(tr.AdamW(1e-3))
    monkeypatch.setenv("GPU_MAX_HW_QUEUES", "4")
    assert callable(tr.make_train_step(tr.AdamW(1e-3)))


def test_graceful_stop_turns_sigterm_and_sigint_into_a_flag():
    """train()'s interrupt handling (train.py:556-562): inside GracefulStop a
    SIGTERM or SIGINT only sets the flag the loop checks after each step; the
    previous handlers are back afterwards."""
    import os
    import signal

    from nlearn_amd.train import GracefulStop

    before = {s: signal.getsignal(s) for s in (signal.SIGINT, signal.SIGTERM)}
    for sig in (signal.SIGTERM, signal.SIGINT):
        with GracefulStop() as stop:
            assert not stop.requested
            os.kill(os.getpid(), sig)   # the Python-level handler runs before the next bytecode
            assert stop.requested
        assert {s: signal.getsignal(s) for s in before} == before


def test_traffic_probe_dispatch_attribution():
    """--traffic-summary attributes PMC rows by dispatch order: GEMM kernels
    take the probe's product tags in launch order (cycling per repetition), a
    split-K reduction joins the GEMM before it, the copy is the calibration,
    and set-up kernels are ignored."""
    import bench

    order = [t for t, _ in bench._traffic_products()]
    assert order[:3] == ["gemm_NN_16384x50257x512", "gemm_NT_16384x512x50257", "gemm_TN_512x50257x16384"]
    assert len(order) == 8 and len(set(order)) == 8 and order[3] == "gemm_NN_9728x50257x512"
    rep = ["void nl::gemm_persist_kernel<true, false, unsigned short, 256, 256, 8, 0>(x)",
           "void nl::gemm2_kernel<256, 256, 64, 2, true, true, unsigned short, 0>(x)",
           "void nl::splitk_reduce_kernel<unsigned short>(x)",
           "void nl::gemm2_kernel<256, 256, 64, 2, false, false, float, 0>(x)",
           "void nl::gemm_persist_kernel<true, false, unsigned short, 256, 256, 8, 0>(x)"]
    for _ in range(4):
        rep += ["void nl::gemm2_kernel<128, 128, 64, 2, false, false, float, 0>(x)",
                "void nl::splitk_reduce_kernel<float>(x)"]
    rep.append("__amd_rocclr_copyBuffer")
    names = ["at::native::normal_kernel(x)"] + rep + rep
    tags = bench._probe_dispatch_tags(names)
    assert tags[0] is None
    one = tags[1:1 + len(rep)]
    assert one == tags[1 + len(rep):]
    assert one[:5] == [order[0], order[1], order[1], order[2], order[3]]
    assert one[5:13] == [t for t in order[4:] for _ in range(2)]
    assert one[-1] == "copy"


def test_lm_head_chunk_bounds():
    """Row chunks of the LM head + CE: two chunks split at 60% of the rows in
    whole 256-row tiles; other counts equal; always covering [0, M) in order."""
    from nlearn_amd.kernels.cross_entropy import chunk_bounds

    assert chunk_bounds(16384, 2) == [0, 9728, 16384]
    assert chunk_bounds(16384, 1) == [0, 16384]
    assert chunk_bounds(16384, 4) == [0, 4096, 8192, 12288, 16384]
    assert chunk_bounds(300, 2) == [0, 150, 300]          # too short for whole tiles
    assert chunk_bounds(3, 16) == [0, 1, 2, 3]
    for M in (1, 255, 512, 777, 4096, 16385):
        for n in (1, 2, 3, 7):
            b = chunk_bounds(M, n)
            assert b[0] == 0 and b[-1] == M and all(x <= y for x, y in zip(b, b[1:]))
