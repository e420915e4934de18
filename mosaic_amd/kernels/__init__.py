"""Drop-in operators with the reference's Python signatures (kernels/*.py of
the reference), each running the gfx950 HIP kernels of ``mosaic_amd``.

Module names mirror the reference modules so call sites change only their
import root.  Every function takes and returns device tensors; none has a CPU
path."""
