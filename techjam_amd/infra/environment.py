"""Environment and GPU-state records for benchmark output.

Same record shape as the reference's ``src/infra/environment.py:41-110``
(cpu, os, python, pytorch, gpu, disk; a clock/power sample; git state), with
ROCm sources in place of ``nvidia-smi``: device properties from torch's HIP
runtime, the amdgpu driver version from sysfs and clocks, power and
temperature from ``rocm-smi``. Every probe is best effort -- a missing tool
gives ``None``, never an exception.
"""

from __future__ import annotations

import json
import os
import platform
import shutil
import subprocess
from pathlib import Path
from typing import Any, Dict, List, Optional


def under_profiler() -> bool:
    """True inside a rocprofv3 run (it exports ROCPROF_* settings). Its
    preloaded library follows every child process and, when counters are
    collected, starts the GPU there before the child's own program runs; a
    child that is a script (``rocm-smi`` starts through ``env python3``) would
    then replace itself after that start. The probes run no tools then."""
    return any(k.startswith("ROCPROF_") for k in os.environ)


def _command_output(command: List[str], timeout: float = 10.0) -> Optional[str]:
    if under_profiler():
        return None
    try:
        done = subprocess.run(command, capture_output=True, text=True, timeout=timeout, check=False)
    except (OSError, subprocess.SubprocessError):
        return None
    if done.returncode != 0:
        return None
    return done.stdout.strip() or None


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _driver_version() -> Optional[str]:
    try:
        return Path("/sys/module/amdgpu/version").read_text().strip() or None
    except OSError:
        return None


def collect_environment(torch_module: Any, device: Any) -> Dict[str, Any]:
    """Host, software and device description of the run."""
    disk = shutil.disk_usage(Path.cwd())
    available = bool(torch_module.cuda.is_available())
    gpu: Dict[str, Any] = {
        "available": available,
        "name": None,
        "arch": None,
        "compute_units": None,
        "total_memory_bytes": None,
        "driver": None,
        "hip_runtime": getattr(torch_module.version, "hip", None),
    }
    if getattr(device, "type", None) == "cuda" and available:
        props = torch_module.cuda.get_device_properties(device)
        gpu["name"] = props.name
        gpu["arch"] = getattr(props, "gcnArchName", None)
        gpu["compute_units"] = props.multi_processor_count
        gpu["total_memory_bytes"] = props.total_memory
        gpu["driver"] = _driver_version()
    return {
        "cpu": _cpu_model(),
        "cpu_count": os.cpu_count(),
        "os": platform.platform(),
        "python": platform.python_version(),
        "pytorch": torch_module.__version__,
        "gpu": gpu,
        "disk": {"path": os.fspath(Path.cwd()), "total_bytes": disk.total, "free_bytes": disk.free},
    }


def collect_gpu_state(device: Any) -> Optional[Dict[str, Any]]:
    """Clocks, power and temperature of the device at this moment
    (``rocm-smi --json``), or ``None`` when unavailable."""
    if getattr(device, "type", None) != "cuda":
        return None
    index = device.index or 0
    text = _command_output(["rocm-smi", "-d", str(index), "--showclocks", "--showpower",
                            "--showtemp", "--json"])
    if not text:
        return None
    try:
        data = json.loads(text[text.index("{"):])
    except (ValueError, json.JSONDecodeError):
        return None
    cards = [v for k, v in data.items() if k.startswith("card") and isinstance(v, dict)]
    return cards[0] if cards else None


def collect_git(root: Optional[Path] = None) -> Dict[str, Any]:
    """Commit and dirtiness of the working tree (``None`` outside a repository)."""
    cwd = os.fspath(root or Path(__file__).resolve().parents[2])
    commit = _command_output(["git", "-C", cwd, "rev-parse", "HEAD"])
    status = _command_output(["git", "-C", cwd, "status", "--short"]) if commit else None
    return {"commit": commit, "dirty": bool(status), "status": status or ""}
