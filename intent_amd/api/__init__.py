from .definitions import Definition, DefinitionKind, HelperDefinition, KernelDefinition, fn, kernel

__all__ = ["Definition", "DefinitionKind", "HelperDefinition", "KernelDefinition", "fn", "kernel"]
