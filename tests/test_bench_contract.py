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
                 "ngdn_param_grads.1", "ngdn_read_state_bwd.2", "ngdn_output_bwd", "ngdn_l0_bwd",
                 "ngdn_promote_chain_fwd.1", "ngdn_output_l0_fwd", "ngdn_output_upper_fwd"):
        nbytes, design, flops = model[name]
        assert 0 < nbytes <= design and flops > 0, name
    # the level-0 intra backward's algorithmic bytes are the op's tensors it
    # touches: reads q0, k, b, v, w (bf16) and g (fp32), writes their
    # gradients: 224 KiB per chunk-head
    assert model["ngdn_l0_bwd_intra"][0] == units * 2 * (5 * 64 * 128 * 2 + 64 * 128 * 4)
    # the fused chunk backward adds the chunk state and its gradient (fp32
    # K x V each), do and mix_0..2 (bf16) to those
    assert model["ngdn_l0_bwd"][0] == units * (2 * (5 * 64 * 128 * 2 + 64 * 128 * 4)
                                               + 2 * 128 * 128 * 4 + 64 * 128 * 2 + 64 * 3 * 2)


def test_step_totals_at_the_headline():
    sys.path.insert(0, ROOT)
    import bench
    from nested_recurrent_memory_amd.inputs import CONFIGS
    nbytes, flops = bench.step_totals(CONFIGS["c2"])
    # op-level tensors once per direction, with fp32 decay and saved states
    assert 5.0e9 < nbytes < 5.6e9
    # dense tile products of the forward and backward
    assert 4.5e11 < flops < 5.5e11
