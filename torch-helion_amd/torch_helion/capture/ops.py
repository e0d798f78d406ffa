"""Op vocabulary of the OpGraph (same names as the reference's
capture/ops.py:22-53, extended additively for the MI355X backend).

* layout ops re-index a tensor and never survive canonicalisation;
* macro ops are model-level patterns the optimizer recognises;
* registered ops are the only ops a fused epilogue may contain.
"""

from __future__ import annotations

LAYOUT_OPS = frozenset({"view", "permute", "expand", "clone", "slice", "cat", "cast"})
BINARY_OPS = frozenset({"add", "sub", "mul", "div", "max", "powf"})
UNARY_OPS = frozenset({"exp", "log", "neg", "rsqrt", "sigmoid", "silu", "tanh", "square", "sqrt", "log1p", "softplus"})
REDUCE_OPS = frozenset({"row_sum", "row_max", "row_mean", "row_sumsq"})
SCAN_OPS = frozenset({"row_cumsum"})
MACRO_OPS = frozenset({"rmsnorm", "rope", "rotate_half", "attention", "softmax", "ssd", "ssd_chunked",
                       "conv1d", "attention_decode", "embedding"})
ANCHOR_OPS = frozenset({"matmul", "batch_matmul", "attention", "attention_decode", "ssd", "ssd_chunked",
                        "conv1d", "embedding"})

REGISTERED_BINARY = frozenset({"add", "sub", "mul", "div", "max", "powf"})
REGISTERED_UNARY = frozenset({"exp", "log"})
REGISTERED_REDUCE = frozenset({"row_sum", "row_max"})
REGISTERED_OPS = REGISTERED_BINARY | REGISTERED_UNARY | REGISTERED_REDUCE | {"matmul", "batch_matmul", "broadcast"}

ELEMENTWISE_OPS = BINARY_OPS | UNARY_OPS

# unregistered unary op -> the registered expression it is rewritten to
UNARY_REWRITES = {
    "log1p": "log(add(x, 1))",
    "softplus": "log(add(1, exp(x)))",
    "neg": "mul(x, -1)",
    "rsqrt": "powf(x, -0.5)",
    "sqrt": "powf(x, 0.5)",
    "sigmoid": "div(1, add(1, exp(mul(x, -1))))",
    "silu": "mul(x, sigmoid(x))",
    "square": "mul(x, x)",
    "tanh": "sub(mul(2, sigmoid(mul(x, 2))), 1)",
}


def is_elementwise(op: str) -> bool:
    return op in ELEMENTWISE_OPS


def is_registered(op: str) -> bool:
    return op in REGISTERED_OPS
