"""torch_mojo_backend (MI355X build): the eager `mojo` device on gfx950.

Public surface as in the reference (torch_mojo_backend/__init__.py):
``register_mojo_devices()`` and ``TorchMojoTensor``; after registration
``model.to("mojo")`` runs the model on the GPU through the hand-written
gfx950 kernel library.  The torch.compile backend of the reference is not
part of this build.
"""

from .mojo_device.register import register_mojo_devices
from .mojo_device.torch_mojo_tensor import TorchMojoTensor

__all__ = ["register_mojo_devices", "TorchMojoTensor"]
