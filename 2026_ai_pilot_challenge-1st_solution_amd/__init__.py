"""MI355X-native batched F-16 air-combat environment hot path.

Drop-in for the reference's GpuDogfight / GpuDogfightVecEnv / BatchObsReward / GAE interfaces,
backed by hand-written gfx950 HIP kernels in libf16hip.so.
"""
from .gpu_env import GpuDogfight, STATE_N, OBS_N, OBS  # noqa: F401
