"""bench.py contract checks that need no GPU: more than one GPU is refused with a
message (each box has one GPU), and --help lists the contract flags."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _run("--gpus", "2", "--steps", "1", "--warmup", "0")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_help_lists_contract_flags():
    r = _run("--help")
    assert r.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in r.stdout


def test_profile_roles_label_the_dispatch_order():
    # a layer step (prefill indexer, top-k, MLA; decode indexer, top-k, MLA with a
    # combine), then a config-3 decode (MLA + combine) and config-4 prefills (MLA
    # with no combine): the labels the counter summary groups the dispatches by
    sys.path.insert(0, ROOT)
    import bench

    names = ["indexer_fp8_kernel", "copy_kernel", "topk_rows_kernel", "mla_w4_kernel", "indexer_fp8_kernel",
             "topk_rows_kernel", "mla_w4_kernel", "mla_combine_kernel", "mla_w4_kernel", "mla_combine_kernel",
             "mla_w4_kernel", "mla_w4_kernel"]
    assert bench._profile_roles(names) == [
        "indexer", None, "topk", "mla", "dec_indexer", "dec_topk", "dec_mla", "dec_mla_combine",
        "config3_mla", "config3_mla_combine", "config4_mla", "config4_mla"]
