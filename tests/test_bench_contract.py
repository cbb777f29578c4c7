"""bench.py's command-line contract that holds without a GPU: this build measures one GPU, so a
request for more exits with a message (and without touching a device); the FLOP helpers that price
the roofline lines count the layers they name."""

from __future__ import annotations

import importlib.util
import os
import subprocess
import sys

from conftest import REPO


def _bench():
    spec = importlib.util.spec_from_file_location("bench_module", REPO / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_exits_with_a_message():
    env = dict(os.environ, HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=120, env=env)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
    assert proc.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="2", HIP_VISIBLE_DEVICES="")
    proc = subprocess.run([sys.executable, str(REPO / "bench.py")], capture_output=True, text=True,
                          timeout=120, env=env)
    assert proc.returncode == 2 and "one GPU" in proc.stderr


def test_config0_flop_count():
    b = _bench()
    # 2 * voxels * cin * cout * 27 taps for the 64^3 x 64 -> 64 headline conv
    assert b.conv_flops(1, 64, 64, 64, 64, 64, 27) == 2 * 64**3 * 64 * 64 * 27 == 57_982_058_496


def test_network_flop_counts_match_the_hand_derivation(ctmr):
    """Config 3's UNet step and config 4's windows, against the per-layer sums worked out by hand for
    the production constructors (conv 2.080 TFLOP with the nearest-2x fold, attention 0.062 TFLOP; one
    20x64x64 decoder window 16.97 TFLOP, four windows 67.87 TFLOP)."""
    b, m = _bench(), ctmr.maisi
    conv, attn = b.unet_flops(m.PRODUCTION_UNET_CONSTRUCTOR, 2, 64, 64, 32)
    assert abs(conv / 1e12 - 2.080) < 0.0015 and abs(attn / 1e12 - 0.0617) < 0.0005
    window = b.vae_decoder_flops(m.PRODUCTION_VAE_CONSTRUCTOR, 20, 64, 64)
    assert abs(window / 1e12 - 16.97) < 0.01 and abs(4 * window / 1e12 - 67.87) < 0.02
