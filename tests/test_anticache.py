"""core.anticache on the CPU: an honest run() passes the three checks, and
each kind of carried state the checks exist for is caught by the check meant
for it (the mistakes are planted in small CPU candidates)."""
import torch

from tilebench_amd.core import anticache as ac


def _maker(shape=(8, 16)):
    seed = [0]

    def make():
        seed[0] += 1
        g = torch.Generator().manual_seed(seed[0])
        return (torch.randn(shape, generator=g), torch.randn(shape[1], 4, generator=g), 3)
    return make


def reference(a, b, k):
    return (a @ b) * k


def _names(res):
    return [(r.name, r.ok) for r in res]


def test_honest_candidate_passes_all_three():
    res = ac.numerical_checks(lambda a, b, k: (a @ b) * k, reference, _maker(), atol=1e-5, rtol=1e-5)
    assert _names(res) == [(n, True) for n in ac.CHECKS]
    assert all(r.mutated_inputs == [] and r.aliased_inputs == [] for r in res)


def test_result_cached_by_address_fails_same_address_new_values():
    cache = {}

    def cand(a, b, k):
        key = (a.data_ptr(), b.data_ptr())
        if key not in cache:
            cache[key] = (a @ b) * k
        return cache[key].clone()

    res = ac.numerical_checks(cand, reference, _maker(), atol=1e-5, rtol=1e-5)
    assert _names(res) == [("fresh_storage", True), ("same_address_new_values", False)]


def test_state_carried_between_calls_fails_repeat():
    calls = [0]

    def cand(a, b, k):
        calls[0] += 1
        y = (a @ b) * k
        return y + 1.0 if calls[0] == 3 else y

    res = ac.numerical_checks(cand, reference, _maker(), atol=1e-5, rtol=1e-5)
    assert _names(res) == [("fresh_storage", True), ("same_address_new_values", True),
                           ("repeat_same_inputs", False)]


def test_input_mutation_is_reported_and_only_allowed_when_declared():
    def cand(a, b, k):
        y = (a @ b) * k
        a.zero_()
        return y

    res = ac.numerical_checks(cand, reference, _maker(), atol=1e-5, rtol=1e-5)
    assert not res[0].ok and res[0].mutated_inputs == [0] and "read-only" in res[0].message
    res = ac.numerical_checks(cand, reference, _maker(), atol=1e-5, rtol=1e-5, mutable=[0])
    assert all(r.ok for r in res) and len(res) == 3


def test_output_aliasing_an_input_fails():
    def cand(a, b, k):
        y = (a @ b) * k
        b.zero_()            # the second output is written into input 1 and returned
        return (y, b)

    def ref(a, b, k):
        return ((a @ b) * k, torch.zeros_like(b))

    res = ac.numerical_checks(cand, ref, _maker(), atol=1e-5, rtol=1e-5, mutable=[1])
    assert not res[0].ok and res[0].aliased_inputs == [1] and "fresh" in res[0].message


def test_nan_inputs_are_not_counted_as_mutated():
    def make():
        a = torch.full((4, 4), float("nan"))
        return (a, torch.ones(4, 4), 1)
    res = ac.numerical_checks(lambda a, b, k: torch.zeros(4, 4), lambda a, b, k: torch.zeros(4, 4), make,
                              atol=0, rtol=0)
    assert all(r.ok and r.mutated_inputs == [] for r in res)
