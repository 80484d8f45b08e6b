"""Decode with two kv heads per workgroup (friday_attn_set_decode_form(·, ·, 1)).

The pair form halves the merge groups, so the split bound doubles and the fp32 additions
happen in another order: its results are held to the decode tolerance against the oracle,
not to the bits of the one-head form. Within the form, the same identities as for the
default form hold bit for bit, and these tests run the default form's own checks with the
pair form switched on: the step against the two-launch sequence (cache rows and rotated q
exact), the int8 step against the three-launch sequence, the fused merge against the merge
kernel, over the reference decode matrix, the benchmark shapes and int8 caches. Shapes
with G > 16 or an odd kv head count keep one kv head per workgroup."""
import pytest

import test_gpu_decode as td
import test_gpu_step as ts

import os

# Built while GPU use was closed: the form has not run on a GPU yet, so the round's
# `pytest -m gpu -x` skips it (a first failure would hide every later test) unless
# FRIDAY_ATTN_TEST_NEW_FORMS=1 asks for it.
pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get("FRIDAY_ATTN_TEST_NEW_FORMS") != "1",
                                 reason="the kv-head pair form has not yet run on a GPU (FRIDAY_ATTN_TEST_NEW_FORMS=1 runs it)")]


@pytest.fixture
def pair(gpu):
    gpu.setDecodeForm(0, 0, 1)
    yield gpu
    gpu.setDecodeForm(-1, -1, -1)


@pytest.mark.parametrize("Hq,Hkv,d,S,max_ctx,neox,devpos", [
    (40, 8, 128, 32768, 32768, 1, True),   # headline
    (32, 8, 128, 8192, 8192, 1, True),     # config 2
    (14, 2, 64, 513, 1024, 1, True),       # config 1
    (32, 8, 128, 1000, 1024, 0, False),    # interleaved pairs, host position
    (40, 8, 128, 1, 64, 1, True),          # first token: one split
])
def test_pair_step(pair, oracle, Hq, Hkv, d, S, max_ctx, neox, devpos):
    print(f"[kv-pair] step {Hq}q/{Hkv}kv d{d} S={S}", flush=True)
    ts.run_step_vs_two_launch(pair, oracle, Hq, Hkv, d, S, max_ctx, 1e6, neox, devpos, seed=S + 3)


@pytest.mark.parametrize("Hq,Hkv,d,S,max_ctx,neox,devpos", [
    (40, 8, 128, 32768, 32768, 1, True),
    (14, 2, 64, 513, 1024, 1, True),
    (40, 8, 128, 1, 64, 1, True),
])
def test_pair_step_q8(pair, oracle, Hq, Hkv, d, S, max_ctx, neox, devpos):
    print(f"[kv-pair] int8 step {Hq}q/{Hkv}kv d{d} S={S}", flush=True)
    ts.test_step_q8_matches_three_launches(pair, oracle, Hq, Hkv, d, S, max_ctx, neox, devpos)


def test_pair_reference_matrix(pair, oracle):
    td.test_reference_decode_matrix(pair, oracle)


@pytest.mark.parametrize("Hq,Hkv,d,S", [(32, 8, 128, 4096), (40, 8, 128, 5000), (16, 16, 128, 333),
                                         (64, 8, 128, 777), (14, 2, 64, 513), (40, 2, 128, 1500)])
def test_pair_shapes(pair, oracle, Hq, Hkv, d, S):
    print(f"[kv-pair] shapes {Hq}q/{Hkv}kv d{d} S={S}", flush=True)
    td.test_shapes(pair, oracle, Hq, Hkv, d, S)


@pytest.mark.parametrize("Hq,Hkv,d,S", [(40, 8, 128, 1000), (14, 2, 64, 513), (10, 2, 128, 60000)])
def test_pair_int8_decode(pair, oracle, Hq, Hkv, d, S):
    print(f"[kv-pair] int8 decode {Hq}q/{Hkv}kv d{d} S={S}", flush=True)
    td.test_int8_decode(pair, oracle, Hq, Hkv, d, S)
