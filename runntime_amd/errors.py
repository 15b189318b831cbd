"""Error types of the MoE ops.

Mirrors src/core/error.ts:3-50 of the reference: a RunntimeError carries one
of the reference's codes; callers check the code, not the message. Argument
checks that the reference makes at graph-build time raise ValueError with
the reference's own message text (src/core/graph/ops/matmul.ts:274-315,
src/core/graph/ops/reduce.ts:93-100), as its plain `Error`s.
"""

RUNNTIME_ERROR_CODES = (
    "LOAD_FAILED",
    "LOAD_ABORTED",
    "CHECKPOINT_MISMATCH",
    "UNSUPPORTED_DEVICE",
    "EXECUTION_FAILED",
    "INVALID_ARGUMENT",
    "RESOURCE_DISPOSED",
    "NOT_INITIALIZED",
)

# moe_status values of include/runntime_moe.h → reference codes.
STATUS_CODES = {
    1: "INVALID_ARGUMENT",
    2: "EXECUTION_FAILED",
    3: "NOT_INITIALIZED",
    4: "RESOURCE_DISPOSED",
}


class RunntimeError(RuntimeError):
    """An error with a `code` from RUNNTIME_ERROR_CODES."""

    def __init__(self, code: str, message: str):
        if code not in RUNNTIME_ERROR_CODES:
            raise ValueError(f"unknown RunntimeError code {code!r}")
        super().__init__(message)
        self.code = code


def is_runntime_error(value, code=None) -> bool:
    """True when `value` is a RunntimeError, with this `code` if one is given
    (error.ts:39-50)."""
    if not isinstance(value, RunntimeError):
        return False
    return code is None or value.code == code
