"""CPU model of the ring GEMM kernels' DMA copies (tests/ring_model/ring_model.cpp).

The model runs the copy plan the kernels compile (go-nngpu_amd/csrc/ring_plan.h) over
every ring configuration the dispatch launches, both operand layouts, ragged M and N, K of
one to three K-tile pairs plus tails, and the refills issued past the end of K: every live
copy must read only elements of its operand and the live copies of a pair must cover the
tile's part of it exactly once. It must also catch the plans it exists for: the fp32 ring
issuing its dead pairs through live descriptors (the plan whose refills read past the end
of K) and the fp16 ring without its per-copy K mask."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MODEL_DIR = os.path.join(ROOT, "tests", "ring_model")
BIN = os.path.join(MODEL_DIR, "_build", "ring_model")
GEMM = os.path.join(ROOT, "go-nngpu_amd", "csrc", "gemm.hip")


@pytest.fixture(scope="module")
def model():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-s", "-C", MODEL_DIR], check=True)
    return BIN


def _run(model, *args):
    return subprocess.run([model, *args], capture_output=True, text=True, timeout=300)


def test_ring_plan_copies_stay_inside_and_cover_each_tile(model):
    r = _run(model)
    assert r.returncode == 0, r.stdout[-3000:]
    m = re.search(r"(\d+) live copies checked, (\d+) violations", r.stdout)
    assert m and int(m.group(2)) == 0
    assert int(m.group(1)) > 5_000_000  # every configuration, layout and shape was walked


def test_model_catches_fp32_dead_pairs_through_live_descriptors(model):
    r = _run(model, "--plant", "f32-dead-pairs-live")
    assert r.returncode == 1
    assert "copy outside the operand" in r.stdout  # the past-the-end reads of that plan


def test_model_catches_fp16_ring_without_k_mask(model):
    r = _run(model, "--plant", "f16-no-kmask")
    assert r.returncode == 1
    assert "VIOLATION" in r.stdout


def test_model_covers_every_ring_launch_in_the_dispatch(model):
    listed = set()
    for line in _run(model, "--list").stdout.splitlines():
        f = line.split()
        listed.add((f[0], int(f[1]), int(f[2]), int(f[3]), int(f[4]), int(f[5])))
    src = open(GEMM).read()
    launched = set()
    for dt, args in re.findall(r"launch_(f16|f32)_ring<([^>]*)>\(", src):
        a = [x.strip() for x in args.split(",")]
        if not a[0].isdigit():
            continue  # the template definitions
        ns = int(a[7]) if len(a) > 7 else 2
        launched.add((dt, int(a[0]), int(a[1]), int(a[2]), int(a[3]), ns))
    # the 32x32x16 NN variant launches its kernel directly: <BM, BN, WM, WN, WPE, NS>, the same
    # copies (F16RingCopies) as the fp16 ring of that tile
    for args in re.findall(r"gemm_f16_ring_mf32_kernel<([^>]*)>\)", src):
        a = [x.strip() for x in args.split(",")]
        if a[0].isdigit():
            launched.add(("f16", int(a[0]), int(a[1]), int(a[2]), int(a[3]), int(a[5])))
    assert launched, "no ring launches found in gemm.hip"
    assert any(x[1:] == (256, 256, 2, 4, 2) for x in launched if x[0] == "f16")
    assert launched <= listed, launched - listed
