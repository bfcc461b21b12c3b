from .artifact import CompiledArtifact, PreparedCall, PreparedRuntime
from .diagnostics import ConfigurationAssessment, NativeObservation, NativeResource
from .interface import PublicInterface, ScalarParameter, StrideSymbol, ViewParameter
from .invocation import BoundPublicArguments, ViewFacts, bind_arguments, invocation_result
from .sequence import PreparedSequence

__all__ = ["CompiledArtifact", "PreparedCall", "PreparedRuntime", "ConfigurationAssessment",
           "NativeObservation", "NativeResource", "PublicInterface", "ScalarParameter",
           "StrideSymbol", "ViewParameter", "BoundPublicArguments", "ViewFacts", "bind_arguments",
           "invocation_result", "PreparedSequence"]
