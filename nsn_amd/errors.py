"""Exception types of the reference's hot path.

The reference raises ``NumericalFailure`` for nonfinite inputs, metadata,
intermediates or outputs and ``IntegrityError`` / ``ContractError`` for
structural problems (experiments/ac08/source/loop_kv_pilot.py:51-60,
experiments/ac08/source/loop_kv_qk01_contract.py:12).  The names are kept so
callers' except clauses work unchanged.
"""


class IntegrityError(RuntimeError):
    pass


class NumericalFailure(RuntimeError):
    pass


class ContractError(Exception):
    pass


def require(ok, message):
    """Structural precondition (the reference's ``w.require``)."""
    if not ok:
        raise IntegrityError(message)
