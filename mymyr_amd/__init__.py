"""mymyr_amd: the MI355X-native state-expansion path of maichmueller/mymyr.

Host C++ (task compiler, drivers) and hand-written HIP kernels for gfx950 behind the C ABI of include/mymyr_amd.h;
this package is the Python mirror of the reference's entry points for that path:

  Task.from_text_file / Task.from_text       task loading (reference Task::from_text_file)
  search.brfs                                device BrFS (reference search.brfs / cuda.brfs)
  rl.DeviceEnvPool                           batched env step on the device (reference rl.CpuEnvPool / DeviceEnv)
  hip.hash_rows, hip.StateSet                hashing and the device dedup set
  dlpack.DeviceBuffer / DeviceArray          library-owned device arrays exported over DLPack (reference DLArray)
  gen                                        seeded synthetic task generators
"""

from .task import Task  # noqa: F401

__all__ = ["Task"]
