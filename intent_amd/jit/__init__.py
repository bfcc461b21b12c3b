from .kernel import JITKernel, jit

__all__ = ["JITKernel", "jit"]
