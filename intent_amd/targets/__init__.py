from .hip import HipTarget, ResolvedHipTarget
from .provider import EnvironmentCheck, LocalExecution, Provider, provider

__all__ = ["HipTarget", "ResolvedHipTarget", "EnvironmentCheck", "LocalExecution", "Provider", "provider"]
