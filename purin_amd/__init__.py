"""MI355X-native Chambolle--Pock projection (PURIN's CP path) on hand-written HIP kernels.

Public names follow the reference package (src/purin/__init__.py:6-45) for the
Chambolle--Pock path.  Names needing torch / the HIP library are imported
lazily so that ``import purin_amd`` works on machines without a GPU.
"""

from importlib import import_module

__version__ = "0.1.0"

_EXPORTS = {
    "Projection": ("problems", "Projection"),
    "ParametricQP": ("problems", "ParametricQP"),
    "ParametricLP": ("problems", "ParametricLP"),
    "MatrixProblem": ("problems", "MatrixProblem"),
    "ChambollePockConfig": ("config", "ChambollePockConfig"),
    "LinearSolverConfig": ("config", "LinearSolverConfig"),
    "ImplicitGradientConfig": ("config", "ImplicitGradientConfig"),
    "SolveStatus": ("types", "SolveStatus"),
    "ProjectionMethod": ("types", "ProjectionMethod"),
    "ProjectionResult": ("types", "ProjectionResult"),
    "ProjectionInfo": ("types", "ProjectionInfo"),
    "ProjectionTrainingOutput": ("types", "ProjectionTrainingOutput"),
    "prepare_projection": ("projection", "prepare_projection"),
    "registered_methods": ("projection", "registered_methods"),
    "Distance": ("projection", "Distance"),
    "WeightedDistance": ("projection", "WeightedDistance"),
    "ChambollePockProjection": ("projection", "ChambollePockProjection"),
    "Plan": ("plan", "Plan"),
    "FunctionalProblem": ("local_quadratic", "FunctionalProblem"),
    "LocalQuadratic": ("local_quadratic", "LocalQuadratic"),
    "QPStructure": ("diagonal_qp", "QPStructure"),
    "QPData": ("diagonal_qp", "QPData"),
}
__all__ = list(_EXPORTS)


def __getattr__(name):
    if name in _EXPORTS:
        module, symbol = _EXPORTS[name]
        value = getattr(import_module("purin_amd." + module), symbol)
        globals()[name] = value
        return value
    raise AttributeError(name)
