"""Plan policies and execution-plan diagnostics.

The single-device build keeps the reference's user-facing planning surface
(reference: src/torch_einshard/symbolic.py:191-289 for ``PlanPolicy`` and the
policy context, :392-445 for ``ExecutionPlan`` / ``last_plan``):

* ``PlanPolicy`` modes ``training | inference | memory | communication |
  latency`` with the same weights.  On one device no transition plan is ranked,
  so a policy is validated and carried but does not change the arithmetic.
* ``optimize(policy)`` (context manager), ``set_default_policy`` and
  ``resolve_plan_policy(optimize=, policy=)`` resolve the active policy.
* Every executed operation records an ``ExecutionPlan``; ``last_plan()`` returns
  its steps (module-global, not thread-safe — as in the reference).
"""

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass

__all__ = [
    "PlanPolicy",
    "PlanStep",
    "PlanCandidate",
    "ExecutionPlan",
    "optimize",
    "resolve_plan_policy",
    "set_default_policy",
    "get_default_policy",
    "get_optimization_policy",
    "set_last_plan",
    "last_plan",
    "last_candidates",
    "last_alternatives",
]


@dataclass(frozen=True)
class PlanPolicy:
    """Weights used to score alternative transition plans."""

    mode: str = "training"
    forward_byte_weight: int = 1
    backward_byte_weight: int = 1
    peak_element_weight: int = 1
    materialized_element_weight: int = 1
    collective_weight: int = 100
    materialization_weight: int = 200
    base_step_weight: int = 1

    @staticmethod
    def from_mode(mode) -> "PlanPolicy":
        if mode is None or isinstance(mode, PlanPolicy):
            return mode or PlanPolicy()
        try:
            overrides = _MODE_WEIGHTS[mode]
        except (KeyError, TypeError):
            raise ValueError(f"Unknown optimization policy {mode!r}") from None
        return PlanPolicy(mode=mode, **overrides)

    def score(self, cost) -> int:
        """Weighted cost of a candidate: its step, collective and materialisation counts
        at full weight, its byte and element counts weighted per KiB (``cost`` carries
        the reference's cost fields)."""
        counted = (
            (cost.score, self.base_step_weight),
            (cost.collectives, self.collective_weight),
            (cost.materializations, self.materialization_weight),
        )
        per_kib = (
            cost.forward_bytes * self.forward_byte_weight + cost.backward_bytes * self.backward_byte_weight,
            cost.peak_elements * self.peak_element_weight,
            cost.materialized_elements * self.materialized_element_weight,
        )
        return sum(n * w for n, w in counted) + sum(v // 1024 for v in per_kib)


# per-mode overrides of the PlanPolicy defaults (reference symbolic.py:203-240)
_MODE_WEIGHTS = {
    "training": {},
    "inference": {"backward_byte_weight": 0},
    "memory": {
        "peak_element_weight": 64,
        "materialized_element_weight": 64,
        "collective_weight": 50,
        "materialization_weight": 400,
    },
    "communication": {
        "forward_byte_weight": 8,
        "backward_byte_weight": 8,
        "collective_weight": 50,
        "materialization_weight": 100,
    },
    "latency": {
        "collective_weight": 1000,
        "materialization_weight": 100,
    },
}

_context_policy: ContextVar = ContextVar("torch_einshard_plan_policy", default=None)
_default_policy = None


def _as_policy(value) -> PlanPolicy:
    return value if isinstance(value, PlanPolicy) else PlanPolicy.from_mode(value)


def resolve_plan_policy(optimize=None, policy=None) -> PlanPolicy:
    if optimize is not None and policy is not None:
        raise ValueError("Pass either optimize or policy, not both")
    if policy is not None:
        return _as_policy(policy)
    if optimize is not None:
        return _as_policy(optimize)
    active = _context_policy.get()
    if active is not None:
        return active
    if _default_policy is not None:
        return _default_policy
    return PlanPolicy()


@contextmanager
def optimize(policy):
    """Make ``policy`` the active plan policy inside the ``with`` block."""
    token = _context_policy.set(_as_policy(policy))
    try:
        yield
    finally:
        _context_policy.reset(token)


def set_default_policy(policy) -> None:
    global _default_policy
    _default_policy = None if policy is None else _as_policy(policy)


def get_default_policy() -> PlanPolicy:
    return _default_policy if _default_policy is not None else PlanPolicy()


def get_optimization_policy() -> PlanPolicy:
    return resolve_plan_policy()


@dataclass(frozen=True)
class PlanStep:
    name: str
    args: tuple = ()


@dataclass(frozen=True)
class PlanCandidate:
    """A strategy an operation weighed, and what became of it (``status``:
    considered / accepted / rejected / ranked / selected, with a ``reason``).  A frozen
    dataclass with the reference's fields (symbolic.py:147-156): callers compare,
    hash and inspect candidates with ``dataclasses`` as they do there."""

    name: str
    args: tuple = ()
    fallback_steps: tuple = ()
    status: str = "considered"
    reason: str = ""

    def with_result(self, status, reason=""):
        """The same candidate with a new status and reason."""
        return PlanCandidate(self.name, self.args, self.fallback_steps, status, reason)


class ExecutionPlan:
    """The record of one operation: the steps it ran, in order, plus the
    candidates it weighed and the alternatives it ranked.  Method names and
    arguments are the reference's (symbolic.py:392-421)."""

    def __init__(self):
        self.steps, self.candidates, self.alternatives = [], [], []

    def add(self, name, *args):
        """Note that step ``name`` ran with ``args``."""
        self.steps.append(PlanStep(name, args))

    def execute(self, name, fn, *fn_args, step_args=(), **fn_kwargs):
        """Note step ``name`` (with ``step_args``), then run ``fn``."""
        self.steps.append(PlanStep(name, tuple(step_args)))
        return fn(*fn_args, **fn_kwargs)

    def consider(self, candidate, *args, status="considered", reason="", fallback_steps=()):
        if not isinstance(candidate, PlanCandidate):
            candidate = PlanCandidate(candidate, tuple(args), tuple(fallback_steps))
        self.candidates.append(candidate.with_result(status, reason))

    def rank(self, alternatives, selected=None, reason=""):
        """Keep ``alternatives``, the one named ``selected`` marked as chosen."""
        self.alternatives = [
            option.with_result("selected", reason) if option.name == selected else option for option in alternatives
        ]

    def names(self):
        return [step.name for step in self.steps]

    def snapshot(self):
        return tuple(self.steps)


# The last operation's record: (steps, candidates, alternatives).  One module-level
# value, replaced whole by each operation (not thread-safe, as in the reference).
_record = ((), (), ())


def set_last_plan(plan):
    """Publish ``plan`` (an ExecutionPlan, or a sequence of steps) as the last one run."""
    global _record
    if isinstance(plan, ExecutionPlan):
        _record = (tuple(plan.steps), tuple(plan.candidates), tuple(plan.alternatives))
    else:
        _record = (tuple(plan), (), ())


def last_plan():
    return _record[0]


def last_candidates():
    return _record[1]


def last_alternatives():
    return _record[2]
