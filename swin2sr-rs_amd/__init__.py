"""swin2sr on MI355X (gfx950): the crate's device backend as hand-written HIP.

Layout of this package:
  csrc/            the HIP kernels and the C ABI (include/swin2sr_hip.h)
  Makefile         builds libswin2sr_hip.so with hipcc --offload-arch=gfx950
  abi.py           ctypes binding of the ABI and the `Backend` mirror (HipBackend)
  model.py         architectures, synthetic checkpoints (crate tensor names) and inputs
  tiling.py        the crate's tile loop and memory policy over the Backend interface
  formats.py       the crate's on-disk formats: converted-checkpoint safetensors with the
                   __metadata__ validation, SW2F golden fixtures, PNG IO

The directory name is not an identifier, so callers load it with
`load_package()` from the repository root (see __graft_entry__.py).
"""
from . import model  # noqa: F401
from . import hip  # noqa: F401
from . import tiling  # noqa: F401
from . import formats  # noqa: F401
from .abi import HipBackend, S2SError, device_info, load_library  # noqa: F401
