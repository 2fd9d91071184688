"""CPU checks of the benchmark's own inputs: the counter summaries its line reads, and the
one-GPU guard. No GPU is touched."""

import fnmatch
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402  (after the path set-up)


def _ignored(path: Path) -> bool:
    """Whether a line of .gpurunignore (tar exclude patterns) drops ``path`` from the tree that
    runs on the GPU machine: a bare pattern matches a file name at any depth, ``./x`` the path
    from the root (and everything below it)."""
    rel = path.relative_to(ROOT).as_posix()
    for line in (ROOT / ".gpurunignore").read_text().splitlines():
        pat = line.strip()
        if not pat or pat.startswith("#"):
            continue
        if pat.startswith("./"):
            p = pat[2:]
            if fnmatch.fnmatch(rel, p) or rel.startswith(p.rstrip("/") + "/"):
                return True
        elif any(fnmatch.fnmatch(part, pat) for part in rel.split("/")):
            return True
    return False


def test_traffic_summaries_are_read_and_travel():
    """The HBM bytes per launch the bench line carries come from committed counter summaries
    that ship with the tree (a summary named *.md would be left behind and read as null)."""
    swiglu = bench.profiled_traffic()
    trunk = bench.profiled_traffic(bench.ATTENTION_TRAFFIC_PROFILE, "traffic_bytes_per_launch_trunk")
    pixel = bench.profiled_traffic(bench.ATTENTION_TRAFFIC_PROFILE, "traffic_bytes_per_launch_pixel")
    # at least the algorithmic bytes of each launch: operands read once, output written once
    assert swiglu >= (4352 * 2560 + 13652 * 2560 + 4352 * 6826) * 2
    assert trunk >= (20 * 4352 * 128 + 2 * 5 * 4352 * 128 + 4352 * 2560) * 2
    assert pixel >= 4 * 10 * 4096 * 128 * 2
    for path in (bench.TRAFFIC_PROFILE, bench.ATTENTION_TRAFFIC_PROFILE):
        assert not _ignored(path), f"{path.name} is excluded from the GPU run's tree"


def test_step_flops_of_the_benchmarked_workload():
    """22.61 TFLOP per 1024x1024 step with 256 text tokens, as the engine computes it (the pixel
    stage's attention projection folded into expand; the figure the line divides by)."""
    from iris_mi355x.config import IRIS_3B

    total = bench.step_flops(IRIS_3B, 1024, 1024, 256)["total"]
    assert abs(total / 1e12 - 22.61) < 0.01


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert res.returncode == 2
    assert "one GPU" in json.loads(res.stdout.strip().splitlines()[-1])["error"]
