"""CPU checks of bench.py's contract that need no GPU: more than one GPU is
refused with a message, and the work model's per-entry-point algorithmic
figures are positive for the headline configuration."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, cwd=ROOT, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in r.stderr


def test_work_model_covers_every_headline_entry_point():
    sys.path.insert(0, ROOT)
    import bench
    from nested_recurrent_memory_amd.inputs import CONFIGS
    model, units = bench.work_model(CONFIGS["c2"])
    assert units == 4 * 16 * 128
    for name in ("ngdn_l0_intra_fwd", "ngdn_l0_scan_fwd", "ngdn_output_fwd", "ngdn_l0_bwd_intra",
                 "ngdn_l0_bwd_state", "ngdn_l0_scan_bwd", "ngdn_probe_fwd.1", "ngdn_probe_bwd.2",
                 "ngdn_param_grads.1", "ngdn_read_state_bwd.2", "ngdn_output_bwd"):
        nbytes, flops = model[name]
        assert nbytes > 0 and flops > 0, name
