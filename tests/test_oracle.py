"""The CPU oracle pinned: conversions against numpy / torch, every check of oracle_checks on the oracle, and each
planted mistake (a mutant build of the oracle) caught by at least one of those checks."""
import numpy as np
import pytest

import oracle_checks as C


def test_f16_conversions(oracle):
    L = oracle.lib()
    # every half bit pattern widens as numpy widens it
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([L.oracle_f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32)[~np.isnan(got)],
                                  want[::7].view(np.uint32)[~np.isnan(want[::7])])
    # narrowing: round to nearest even, subnormals, overflow, ties
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-8, 6, 3000),
                         np.array([65504, 65519.99, 65520, 6e-8, 2.98e-8, 2.9802322e-8, 5.96e-8, 1e-10, -0.0, 0.0,
                                   1 + 2 ** -11, 1 + 3 * 2 ** -11, np.inf, -np.inf], np.float32)]).astype(np.float32)
    got = np.array([L.oracle_f32_to_f16(float(x)) for x in xs], np.uint16)
    with np.errstate(over="ignore"):
        want16 = xs.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want16)


def test_bf16_conversion_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    L = oracle.lib()
    rng = np.random.default_rng(1)
    xs = np.concatenate([rng.standard_normal(2000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 2000),
                         np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, 3.3895314e38, -0.0], np.float32)]).astype(np.float32)
    want = torch.from_numpy(xs).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([L.oracle_f32_to_bf16(float(x)) for x in xs], np.uint16)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(oracle.to_bf16_bits(xs), want)


@pytest.mark.parametrize("check", C.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_passes(check, oracle):
    ok, msg = check()
    assert ok, msg


MUTANTS = {1: "mask off by one", 2: "GQA map h % kv_heads", 3: "lse without the maximum",
           4: "k and v swapped in the scores", 5: "cube_topk ties to the larger index",
           6: "sparse dense rows ignore valid", 7: "heads rotation sign of the second value",
           8: "heads norm divides by the sum", 9: "gathered lists read past count",
           10: "probabilities not rounded to half", 11: "proj x not rounded to bf16",
           12: "proj weight transposed", 13: "kda read before the decay", 14: "kda beta not applied"}


@pytest.mark.parametrize("mutant", sorted(MUTANTS), ids=lambda m: MUTANTS[m].replace(" ", "_"))
def test_planted_mistake_is_caught(mutant, oracle):
    failed = [c.__name__ for c in C.ALL_CHECKS if not c(mutant=mutant)[0]]
    assert failed, f"no check catches the planted mistake: {MUTANTS[mutant]}"
