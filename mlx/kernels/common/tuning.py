# Per-chip dispatch overrides. Key: (kernel, chip) -> {threadgroup, grid}.
# Fallback: exact chip -> generation -> registry default (same mechanism as
# reference mlx/kernels/common/tuning.py:1-6).  On gfx950 the HIP kernels
# derive their launch from the scalars, so an override only changes the
# advisory geometry the report prints.

CHIP_TUNING: dict[tuple[str, str], dict] = {}
