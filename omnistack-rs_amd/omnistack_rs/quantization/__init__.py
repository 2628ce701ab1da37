from omnistack_rs.quantization.codebook import (
    LloydMaxCalibrator,
    calibrate_codebook,
    calibrate_heads,
    calibrate_per_group,
)
from omnistack_rs.quantization.qjl import RademacherQJL, qjl_encode, qjl_reconstruct

__all__ = [
    "LloydMaxCalibrator",
    "calibrate_codebook",
    "calibrate_per_group",
    "calibrate_heads",
    "RademacherQJL",
    "qjl_encode",
    "qjl_reconstruct",
]
