"""Measurement scripts: kernel timing beside the platform libraries (`compare_libs`) and the per-kernel launch
sequence that rocprofv3 counter runs profile (`profile_kernels`). Run as `python -m foidfinder_amd.measure.<name>`;
nothing on the served path imports this package."""
