"""The eager `mojo` PrivateUse1 device."""
