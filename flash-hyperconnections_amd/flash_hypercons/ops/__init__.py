from .matrix_exp import matrix_exp, use_backend  # noqa: F401
