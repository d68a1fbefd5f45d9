"""CPU tensors that report a HIP device, for tests of host-side logic that
checks a tensor's device before it hands the pointer to a kernel (entry
builders, argument checks). Nothing here reaches a GPU."""


class _Dev:
    def __init__(self, index):
        self.index = index
        self.type = "cuda"

    def __repr__(self):
        return f"cuda:{self.index}"


class FakeDeviceTensor:
    """A CPU tensor that reports itself as on device ``index``."""
    is_cuda = True

    def __init__(self, t, index=0):
        self._t = t
        self.device = _Dev(index)

    def __getattr__(self, name):
        return getattr(self._t, name)
