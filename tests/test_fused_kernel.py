"""GPU parity and behaviour tests of the HIP sampler (libfsamp.so through fused_sampling).

Mirrors the reference's tests/test_fused_kernel.py (cited per test) with the CPU oracle
(oracle/fsamp_oracle.c) in place of benchmarks/reference.py.  The oracle's fp32 tail fixes
the same evaluation order as the kernel's, so candidate ids, keep masks, renormed
probabilities and token ids are compared bit for bit, not within a tolerance.
"""

import math
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from llm_sampling_kernel_amd import _lib, fused, fused_sampling  # noqa: E402
from llm_sampling_kernel_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402

import cabi  # noqa: E402

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
DTYPES = ["float16", "bfloat16"]
TORCH_DTYPE = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def dev(bits: np.ndarray, dtype: str) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    return t.view(TORCH_DTYPE[dtype]).cuda()


def bits_of(x: torch.Tensor) -> np.ndarray:
    return x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def randn_bits(shape, seed, scale, dtype):
    x = np.random.Generator(np.random.PCG64(seed)).standard_normal(shape).astype(np.float32)
    return W.to_bits(x * scale, dtype)


def ustream(B, seed):
    return np.random.Generator(np.random.PCG64(seed)).random(B, dtype=np.float32)


def oracle(bits, dtype, k, p, u):
    return O.sample(bits, dtype, k, p, u, return_stages=True, nthreads=8)


def run_u(x, k, p, u_np, splits=0):
    u = torch.from_numpy(u_np).cuda()
    tok = fused.sample_fused_u(x, k, p, u, splits)
    ids, keep, ren = fused_sampling.stages_fused_u(x, k, p, u, splits)
    torch.cuda.synchronize()
    return tok.cpu().numpy(), ids.cpu().numpy(), keep.cpu().numpy(), ren.cpu().numpy()


def rank_of(topk_ids, tok):
    return (topk_ids == tok[:, None]).argmax(-1)


def test_the_sampler_runs_from_the_in_tree_hip_library():
    lib = _lib.load()
    assert os.path.dirname(os.path.abspath(lib._name)) == os.path.dirname(_lib.__file__)
    x = torch.zeros(2, 64, device="cuda", dtype=torch.bfloat16)
    assert fused.topk_fused(x, 3).tolist() == [[0, 1, 2]] * 2


# --- the five benchmark configurations, full size ---------------------------------------------

FIX = np.load(os.path.join(HERE, "golden", "workloads.npz"))


@pytest.mark.parametrize("name", W.CASE_NAMES)
def test_workload_parity_with_the_golden_fixture_and_the_oracle(name):
    c = W.case(name)
    assert c.digest() == bytes(FIX[f"{name}/digest"]).decode(), "seeded inputs differ"
    x = dev(c.logits, c.dtype)
    ids = fused.topk_fused(x, c.top_k).cpu().numpy()
    assert np.array_equal(ids, FIX[f"{name}/topk_ids"]), "candidate set or order differs"
    tok, _, keep, ren = run_u(x, c.top_k, c.top_p, c.u)
    assert np.array_equal(tok, FIX[f"{name}/token_ids"]), "token ids differ"
    assert np.array_equal(keep.sum(-1), FIX[f"{name}/cutoff"]), "nucleus size differs"
    s = oracle(c.logits, c.dtype, c.top_k, c.top_p, c.u)
    assert np.array_equal(ren.view(np.uint32), s.renormed.view(np.uint32)), "renormed bits differ"
    # retained mass against fp64: within 1e-5 relative
    p64, c64, _, cut64 = O.stages_f64(c.logits, c.dtype, c.top_k, c.top_p)
    zp = s.cumsum[np.arange(c.batch), s.cutoff - 1].astype(np.float64)
    z64 = c64[np.arange(c.batch), cut64 - 1]
    same = s.cutoff == cut64
    assert same.mean() >= 0.95
    assert (np.abs(zp - z64)[same] / z64[same]).max() < 1e-5


def test_c5_properties_at_full_batch():
    c = W.c5()
    x = dev(c.logits, c.dtype)
    ids = fused.topk_fused(x, 50)
    # sortedness (non-increasing value along the row) and ids address their own values
    vals = torch.gather(x.float(), 1, ids)
    assert (vals[:, :-1] >= vals[:, 1:]).all()
    assert (vals[:, -1:] >= x.float()).sum(-1).ge(50).all()
    # idempotence: sampling twice with the same u gives the same tokens
    u = torch.from_numpy(c.u).cuda()
    assert torch.equal(fused.sample_fused_u(x, 50, 0.9, u), fused.sample_fused_u(x, 50, 0.9, u))


# --- candidate set (reference tests/test_fused_kernel.py:29-45) --------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("top_k", [1, 20, 50, 100, 1024])
@pytest.mark.parametrize("vocab", [2000, 4001, 128256, 151936])
def test_candidate_set_matches_the_oracle_exactly(vocab, top_k, dtype):
    bits = randn_bits((16, vocab), vocab + top_k, 4.0, dtype)
    got = fused.topk_fused(dev(bits, dtype), top_k).cpu().numpy()
    want = oracle(bits, dtype, top_k, 0.9, np.zeros(16, np.float32)).topk_ids
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", DTYPES)
def test_all_equal_logits_resolve_to_the_lowest_token_ids(dtype):
    x = torch.zeros(4, 4000, device="cuda", dtype=TORCH_DTYPE[dtype])
    assert fused.topk_fused(x, 50).tolist() == [list(range(50))] * 4


def test_plus_and_minus_zero_tie():
    bits = np.array([[0x8000, 0x0000, 0x8000, 0x3F80, 0x0000, 0xBF80, 0x8000, 0x0000]], np.uint16)
    x = dev(bits, "bfloat16")
    assert fused.topk_fused(x, 8).tolist() == [[3, 0, 1, 2, 4, 6, 7, 5]]


@pytest.mark.parametrize("vocab,splits", [(151936, 1), (151936, 8), (20000, 4), (5000, 1)])
def test_ties_past_the_candidate_buffer_are_still_exact(vocab, splits):
    # reference :132-141 -- every element ties, far more than the LDS candidate buffer holds
    x = torch.zeros(2, vocab, device="cuda", dtype=torch.bfloat16)
    for top_k in (1, 50, 100, 1024):
        assert fused.topk_fused(x, top_k, splits=splits).tolist() == [list(range(top_k))] * 2


@pytest.mark.parametrize("vocab", [20000, 151936])
def test_dense_tie_rows_match_the_oracle_with_one_split(vocab):
    # reference :144-151
    bits = randn_bits((8, vocab), 44, 0.05, "bfloat16")
    x = dev(bits, "bfloat16")
    for top_k in (20, 50, 100, 1024):
        want = oracle(bits, "bfloat16", top_k, 0.9, np.zeros(8, np.float32)).topk_ids
        assert np.array_equal(fused.topk_fused(x, top_k, splits=1).cpu().numpy(), want)


def test_tie_grid_rows_through_every_path():
    # 64-value grid (C3-like) at every split count: filter path and radix fallback agree
    c = W.c3()
    x = dev(c.logits, c.dtype)
    want = FIX["C3/topk_ids"]
    for s in (1, 2, 3, 4, 8, 16, 32, 64):
        assert np.array_equal(fused.topk_fused(x, 50, splits=s).cpu().numpy(), want), s


@pytest.mark.parametrize("shift, scale", [(-20.0, 1.0), (1.0, 0.25), (0.0, 3.0)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_candidate_sort_matches_the_oracle_on_either_side_of_its_32_bit_form(shift, scale, dtype):
    # up to 64 candidates are sorted as 32-bit words when the bound's key is >= 0xC000 (rows
    # whose top values are at least 2.0); all-negative rows and rows of small values take the
    # 64-bit words instead.  Both must give the oracle's candidates, order and tokens.
    x32 = np.random.Generator(np.random.PCG64(91)).standard_normal((6, 50000)).astype(np.float32)
    bits = W.to_bits(x32 * scale + shift, dtype)
    x = dev(bits, dtype)
    u = ustream(6, 92)
    want = oracle(bits, dtype, 50, 0.9, u)
    tok, _, keep, ren = run_u(x, 50, 0.9, u)
    assert np.array_equal(fused_sampling.topk_fused(x, 50, 0).cpu().numpy(), want.topk_ids)
    assert np.array_equal(tok, want.token_ids)
    assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32))


@pytest.mark.parametrize("k", [129, 200, 257, 511, 513, 1000])
def test_split_rows_with_wide_k_merge_in_the_workgroup_exactly(k):
    # k > 128 with split rows takes the workgroup hand-off and merge (merge widths 256, 512
    # and 1024, k not a power of two): candidates, order, tokens and renormed bit-exact
    bits = randn_bits((3, 151936), 95 + k, 2.0, "bfloat16")
    x = dev(bits, "bfloat16")
    u = ustream(3, 96)
    want = oracle(bits, "bfloat16", k, 0.99, u)
    for s in (0, 2, 3):
        tok, _, keep, ren = run_u(x, k, 0.99, u, s)
        assert np.array_equal(fused_sampling.topk_fused(x, k, s).cpu().numpy(), want.topk_ids), s
        assert np.array_equal(tok, want.token_ids), s
        assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32)), s


@pytest.mark.parametrize("k", [300, 1000])
def test_wide_selection_falls_back_where_its_key_bins_do_not_reach(k):
    # Split rows with k > 256 rank their candidates in key bins below the slice maximum and
    # merge the lists the same way.  Row 0: split 0 holds 100 values near +8 and otherwise
    # -1e4, the other splits values near -50 -- split 0's bound lies past the bins (its slice
    # falls back to the general selection) and the merged top k mostly lies past the bins of
    # the row maximum (the merge falls back to the bitonic merge).  Row 1: values spread over
    # many binades (the bound lies past the bins in every slice).  Row 2: ordinary values.
    B, V = 3, 151936
    g = np.random.Generator(np.random.PCG64(4100 + k))
    x32 = np.empty((B, V), np.float32)
    x32[0] = -50.0 + g.standard_normal(V)
    x32[0, :V // 4] = -1.0e4 + g.standard_normal(V // 4)
    x32[0, :100] = 8.0 + g.standard_normal(100)
    x32[1] = np.sign(g.standard_normal(V)) * np.exp2(g.uniform(-60.0, 60.0, V))
    x32[2] = 3.0 * g.standard_normal(V)
    bits = W.to_bits(x32, "bfloat16")
    x = dev(bits, "bfloat16")
    u = ustream(B, 4200 + k)
    want = oracle(bits, "bfloat16", k, 0.99, u)
    for s in (0, 4):
        tok, _, keep, ren = run_u(x, k, 0.99, u, s)
        assert np.array_equal(fused_sampling.topk_fused(x, k, s).cpu().numpy(), want.topk_ids), s
        assert np.array_equal(tok, want.token_ids), s
        assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32)), s


def test_vocabularies_past_18_bit_ids_keep_the_exact_order():
    # ids of 2^18 and more do not fit the 32-bit sort words: those slices sort 64-bit words
    V = (1 << 18) + 4000
    bits = randn_bits((3, V), 93, 3.0, "bfloat16")
    x = dev(bits, "bfloat16")
    u = ustream(3, 94)
    want = oracle(bits, "bfloat16", 50, 0.9, u)
    for s in (0, 1):
        tok, _, keep, ren = run_u(x, 50, 0.9, u, s)
        assert np.array_equal(fused_sampling.topk_fused(x, 50, s).cpu().numpy(), want.topk_ids), s
        assert np.array_equal(tok, want.token_ids), s
        assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32)), s


def test_every_split_count_and_workgroup_size_gives_the_same_answer():
    bits = randn_bits((4, 151936), 45, 3.0, "bfloat16")
    x = dev(bits, "bfloat16")
    u = ustream(4, 46)
    want = oracle(bits, "bfloat16", 50, 0.9, u)
    ud = torch.from_numpy(u).cuda()
    for threads in (0, 256, 512, 1024):
        for s in (1, 2, 5, 8, 19, 32, 81):
            try:
                tok, keep, ren = cabi.run(x, 50, 0.9, u=ud, splits=s, threads=threads,
                                          stages=True)
            except _lib.FsampError as e:
                assert e.status == 10  # this size cannot tile the slice: a clean refusal
                continue
            assert np.array_equal(tok.cpu().numpy(), want.token_ids), (threads, s)
            assert np.array_equal(ren.cpu().numpy().view(np.uint32),
                                  want.renormed.view(np.uint32))


# --- sampling (reference :48-108) ---------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("top_p", [0.5, 0.90, 0.95, 1.0])
def test_sampled_token_is_inside_the_oracle_nucleus(top_p, dtype):
    bits = randn_bits((8, 151936), 50, 4.0, dtype)
    x = dev(bits, dtype)
    s = oracle(bits, dtype, 50, top_p, np.zeros(8, np.float32))
    for off in range(32):
        tok = fused.sample_fused(x, 50, top_p, offset=off).cpu().numpy()
        hit = s.topk_ids == tok[:, None]
        assert hit.any(-1).all()
        assert (rank_of(s.topk_ids, tok) < s.cutoff).all()
        # and exactly the oracle's draw for the same splitmix64 uniforms
        u = O.rng_uniform(fused.DEFAULT_SEED, off, 8)
        assert np.array_equal(tok, oracle(bits, dtype, 50, top_p, u).token_ids)


def test_top_k_one_is_the_argmax_and_ignores_the_rng():
    bits = randn_bits((8, 4000), 51, 4.0, "bfloat16")
    x = dev(bits, "bfloat16")
    expected = x.float().argmax(dim=-1)
    for off in range(8):
        assert torch.equal(fused.sample_fused(x, 1, 0.9, offset=off), expected)


def test_one_hot_logits_always_sample_the_spike():
    x = torch.full((8, 4000), -30.0, device="cuda", dtype=torch.bfloat16)
    x[:, 1234] = 30.0
    for off in range(8):
        assert (fused.sample_fused(x, 50, 0.9, offset=off) == 1234).all()


def test_sampling_frequencies_match_the_renormalized_distribution():
    probs = [0.40, 0.30, 0.15, 0.10, 0.05]
    n = 20000
    row = torch.log(torch.tensor(probs, device="cuda"))
    x = row.expand(n, 5).contiguous().to(torch.bfloat16)
    tok = fused.sample_fused(x, 5, 1.0, offset=0).cpu().numpy()
    s = oracle(bits_of(x), "bfloat16", 5, 1.0, np.zeros(n, np.float32))
    freq = np.bincount(rank_of(s.topk_ids, tok), minlength=5) / n
    assert np.abs(freq - s.renormed[0]).max() < 4 * math.sqrt(0.4 * 0.6 / n)


def test_equal_logits_sample_close_to_uniform():
    k, n = 8, 4096
    x = torch.zeros(n, k, device="cuda", dtype=torch.bfloat16)
    counts = torch.bincount(fused.sample_fused(x, k, 1.0, offset=0), minlength=k).float()
    assert (counts > 0).all()
    sigma = math.sqrt(n * (1 / k) * (1 - 1 / k))
    assert (counts - n / k).abs().max().item() < 4 * sigma


def test_the_top_p_cutoff_matches_the_oracle_cutoff():
    bits = randn_bits((4, 4000), 52, 2.0, "bfloat16")
    x = dev(bits, "bfloat16")
    s = oracle(bits, "bfloat16", 50, 0.9, np.zeros(4, np.float32))
    seen = np.zeros((4, 50), bool)
    for off in range(4000):
        tok = fused.sample_fused(x, 50, 0.90, offset=off).cpu().numpy()
        seen[np.arange(4), rank_of(s.topk_ids, tok)] = True
    assert np.array_equal(seen.sum(-1), s.cutoff)


def test_same_seed_and_offset_reproduce_and_different_offsets_advance():
    x = dev(randn_bits((64, 4000), 53, 4.0, "bfloat16"), "bfloat16")
    a = fused.sample_fused(x, 50, 0.9, seed=7, offset=3)
    assert torch.equal(a, fused.sample_fused(x, 50, 0.9, seed=7, offset=3))
    assert not torch.equal(a, fused.sample_fused(x, 50, 0.9, seed=7, offset=4))
    assert not torch.equal(a, fused.sample_fused(x, 50, 0.9, seed=8, offset=3))


def test_generator_path_advances_and_reseeding_reproduces():
    x = dev(randn_bits((64, 4000), 54, 4.0, "bfloat16"), "bfloat16")
    torch.manual_seed(123)
    a = fused.sample_fused(x, 50, 0.9)
    b = fused.sample_fused(x, 50, 0.9)
    assert not torch.equal(a, b)
    torch.manual_seed(123)
    assert torch.equal(a, fused.sample_fused(x, 50, 0.9))


def test_rejects_shapes_and_dtypes_outside_the_regime():
    x = torch.randn(2, 4000, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        fused.sample_fused(x.float(), 50, 0.9)
    with pytest.raises(RuntimeError, match=r"top_k must be <= 1024"):
        fused.sample_fused(x, 2000, 0.9)
    with pytest.raises(RuntimeError, match=r"top_k must be >= 1"):
        fused.sample_fused(x, 0, 0.9)
    with pytest.raises(RuntimeError, match=r"top_p must be in \(0, 1\]"):
        fused.sample_fused(x, 50, 1.5)
    with pytest.raises(RuntimeError, match="contiguous cuda"):
        fused.sample_fused(x.t().contiguous().t(), 50, 0.9)
    with pytest.raises(RuntimeError, match="contiguous cuda"):
        fused.sample_fused(x.cpu(), 50, 0.9)


# --- edge shapes ---------------------------------------------------------------------------------

@pytest.mark.parametrize("B,V,k", [(1, 1, 1), (3, 7, 50), (2, 30, 500), (5, 1024, 1024),
                                   (1, 9, 8), (300, 4000, 50), (7, 4001, 100), (2, 100000, 1000)])
def test_edge_shapes_match_the_oracle(B, V, k):
    for dtype in DTYPES:
        bits = randn_bits((B, V), B * 1000 + V, 3.0, dtype)
        x = dev(bits, dtype)
        u = ustream(B, V)
        s = oracle(bits, dtype, k, 0.9, u)
        tok, ids, keep, ren = run_u(x, k, 0.9, u)
        assert np.array_equal(fused.topk_fused(x, k).cpu().numpy(), s.topk_ids)
        assert np.array_equal(tok, s.token_ids)
        assert np.array_equal(keep, s.keep)
        assert np.array_equal(ren.view(np.uint32), s.renormed.view(np.uint32))


def test_unaligned_rows_take_the_element_path():
    bits = randn_bits((4, 20001), 55, 3.0, "bfloat16")
    full = dev(bits.reshape(-1), "bfloat16")
    x = full[1:20001].view(4, 5000)  # starts 2 bytes into an allocation
    assert x.data_ptr() % 16 != 0
    want = oracle(bits_of(x), "bfloat16", 50, 0.9, np.zeros(4, np.float32)).topk_ids
    assert np.array_equal(fused.topk_fused(x, 50).cpu().numpy(), want)


def test_masked_and_extreme_rows():
    x = torch.randn(6, 5000, device="cuda") * 3
    x[0, 100:] = float("-inf")
    x[1, :] = -3e38
    x[1, 7] = -1e38
    x[2, :] = 3e38
    x[3, ::3] = 0.0
    x[4, :] = -0.0
    x[5, 10:] = float("-inf")
    for td in (torch.bfloat16,):
        xx = x.to(td)
        bits = bits_of(xx)
        u = ustream(6, 56)
        s = oracle(bits, "bfloat16", 100, 0.95, u)
        tok, _, keep, ren = run_u(xx, 100, 0.95, u)
        assert np.array_equal(tok, s.token_ids)
        assert np.array_equal(keep, s.keep)
        assert np.array_equal(ren.view(np.uint32), s.renormed.view(np.uint32))
        assert (tok[[0, 5]] < [100, 10]).all()


def test_workspace_is_reused_safely_across_batch_sizes():
    x = dev(randn_bits((256, 8000), 57, 3.0, "bfloat16"), "bfloat16")
    bits = bits_of(x)
    for B in (1, 64, 2, 256, 3, 256, 1):
        want = oracle(bits[:B], "bfloat16", 50, 0.9, np.zeros(B, np.float32)).topk_ids
        assert np.array_equal(fused.topk_fused(x[:B], 50, splits=4).cpu().numpy(), want), B


# --- ablation (reference :164-198) --------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("batch", [1, 8])
def test_the_last_ablation_phase_is_the_production_path(batch, dtype):
    # phase 7 is the whole sampler with seed = offset = 0: the oracle's tokens for the
    # splitmix64 uniforms of (0, 0, row)
    bits = randn_bits((batch, 4000), 58 + batch, 4.0, dtype)
    x = dev(bits, dtype)
    u = O.rng_uniform(0, 0, batch)
    for top_k in (20, 50):
        got = fused_sampling.probe_phase(x, top_k, 0.9, 7, 0).cpu().numpy()
        assert np.array_equal(got, oracle(bits, dtype, top_k, 0.9, u).token_ids)


def test_early_ablation_phases_stop_before_the_answer_exists():
    x = dev(randn_bits((4, 4000), 60, 4.0, "bfloat16"), "bfloat16")
    full = fused_sampling.probe_phase(x, 50, 0.9, 7, 0)
    for phase in (1, 2, 3, 4, 5, 6):
        assert fused_sampling.probe_phase(x, 50, 0.9, phase, 0).shape == full.shape
    six = fused_sampling.probe_phase(x, 50, 0.9, 6, 0)
    assert torch.equal(six, x.float().argmax(-1))


def test_ablation_rejects_phases_outside_the_pipeline():
    x = torch.zeros(2, 4000, device="cuda", dtype=torch.bfloat16)
    for phase in (0, -1, 8):
        with pytest.raises(RuntimeError):
            fused_sampling.probe_phase(x, 50, 0.9, phase, 0)


# --- Gate A (reference :201-257) -----------------------------------------------------------------

@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("top_p", [0.9, 0.95, 1.0])
@pytest.mark.parametrize("top_k", [1, 20, 50, 100])
def test_gate_a_keep_and_renormed_match_the_oracle_bit_for_bit(top_k, top_p, dtype):
    bits = randn_bits((64, 151936), 70 + top_k, 4.0, dtype)
    x = dev(bits, dtype)
    s = oracle(bits, dtype, top_k, top_p, np.zeros(64, np.float32))
    _, keep, ren = fused_sampling.stages_fused(x, top_k, top_p, 0, 0, 0)
    assert np.array_equal(keep.cpu().numpy(), s.keep)
    assert np.array_equal(ren.cpu().numpy().view(np.uint32), s.renormed.view(np.uint32))
    assert (ren.cpu().numpy()[~s.keep] == 0).all()
    # and within the reference's own tolerance of the fp64 restatement
    _, _, r64, _ = O.stages_f64(bits, dtype, top_k, top_p)
    assert np.allclose(ren.cpu().numpy(), r64, atol=2e-6, rtol=0)


def test_gate_a_renormed_sums_to_one_over_the_nucleus():
    x = dev(randn_bits((32, 151936), 80, 4.0, "bfloat16"), "bfloat16")
    for top_p in (0.9, 0.95, 1.0):
        _, _, ren = fused_sampling.stages_fused(x, 50, top_p, 0, 0, 0)
        assert torch.allclose(ren.sum(-1), torch.ones(32, device="cuda"), atol=1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("top_p,expected_kept", [(0.25, 2), (0.5, 4), (0.75, 6), (0.875, 7)])
def test_gate_a_cut_lands_exactly_on_the_boundary(top_p, expected_kept, dtype):
    x = torch.full((4, 4000), -30.0, device="cuda", dtype=TORCH_DTYPE[dtype])
    x[:, :8] = 10.0
    _, keep, _ = fused_sampling.stages_fused(x, 8, top_p, 0, 0, 0)
    assert keep.sum(-1).tolist() == [expected_kept] * 4


# --- graphs (reference :260-308) -----------------------------------------------------------------

def test_graph_replay_with_explicit_uniforms_tracks_the_u_buffer():
    bits = randn_bits((8, 4000), 90, 2.0, "bfloat16")
    x = dev(bits, "bfloat16")
    u = torch.zeros(8, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fused.sample_fused_u(x, 50, 0.95, u)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fused.sample_fused_u(x, 50, 0.95, u)
    for i in range(16):
        un = ustream(8, 100 + i)
        u.copy_(torch.from_numpy(un))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), oracle(bits, "bfloat16", 50, 0.95, un).token_ids)
        assert torch.equal(out, fused.sample_fused_u(x, 50, 0.95, u))


def test_an_explicit_offset_is_still_reproducible():
    x = dev(randn_bits((8, 4000), 91, 2.0, "bfloat16"), "bfloat16")
    a = fused_sampling.sample_fused(x, 50, 0.9, 1234, 7, 0)
    b = fused_sampling.sample_fused(x, 50, 0.9, 1234, 7, 0)
    c = fused_sampling.sample_fused(x, 50, 0.9, 1234, 8, 0)
    assert torch.equal(a, b)
    assert not torch.equal(a, c)


def test_floor_probes_return_the_argmax():
    bits = randn_bits((8, 151936), 92, 3.0, "bfloat16")
    x = dev(bits, "bfloat16")
    want = x.float().argmax(-1)
    assert torch.equal(fused_sampling.probe_scan_rowblock(x), want)
    for s in (1, 8, 35, 70, 140, 280):
        assert torch.equal(fused_sampling.probe_scan_split(x, s), want)
    assert fused_sampling.probe_noop(x).shape == (8,)


@pytest.mark.parametrize("V", [1000, 8 * 1024 * 19 + 8, 128256, 151937])
def test_floor_scan_probe_batches_and_row_ends(V):
    # rows shorter than one batch of vector loads, one vector past a full batch, the C2 row, and
    # a row that is not a multiple of 8 (element loads)
    bits = randn_bits((3, V), 93, 2.0, "float16")
    x = dev(bits, "float16")
    want = x.float().argmax(-1)
    assert torch.equal(fused_sampling.probe_scan_rowblock(x), want)
    assert torch.equal(fused_sampling.probe_scan_split(x, 3), want)


@pytest.mark.parametrize("V", [151936, 128256, 1000])
def test_load_floor_probe_reads_each_waves_share(V):
    # wave w of the 512-thread workgroup owns vectors c*512 + 64w .. c*512 + 64w + 63
    bits = randn_bits((5, V), 94, 3.0, "bfloat16")
    got = fused_sampling.probe_load(dev(bits, "bfloat16")).cpu().numpy().view(np.uint32)
    keys = O.key16(bits).reshape(5, V // 8, 8).max(axis=2)
    owner = (np.arange(V // 8) % 512) // 64
    want = np.stack([keys[:, owner == w].max(axis=1) if (owner == w).any()
                     else np.zeros(5, np.uint32) for w in range(8)], axis=1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("B,V", [(5, 151936), (3, 1000), (1, 8)])
def test_stream_floor_probe_reads_every_block(B, V):
    # workgroup g reads vectors g*1024 + u*256 + t (u < 4, t < 256), the batch's last vector
    # standing in past its end; wave w of g holds the lanes t in [64w, 64w + 64)
    bits = randn_bits((B, V), 95, 3.0, "bfloat16")
    got = fused_sampling.probe_stream(dev(bits, "bfloat16")).cpu().numpy().view(np.uint32)
    vmax = O.key16(bits).reshape(-1, 8).max(axis=1)
    nvec = vmax.size
    groups = (nvec + 1023) // 1024
    assert got.size == groups * 4
    g = np.arange(groups)[:, None, None, None]
    w = np.arange(4)[None, :, None, None]
    u = np.arange(4)[None, None, :, None]
    lane = np.arange(64)[None, None, None, :]
    idx = np.minimum(g * 1024 + u * 256 + w * 64 + lane, nvec - 1)
    want = vmax[idx].reshape(groups, 4, -1).max(axis=2).reshape(-1)
    assert np.array_equal(got, want)
    assert got.max() == O.key16(bits).max()


def test_kernel_attrs_report_every_instantiation_without_spills_in_the_planned_tilings():
    rows = fused_sampling.kernel_attrs()
    # every compiled tiling twice (common, then ",merge"), in the order of the kernel table
    assert len(rows) % 2 == 0 and len(rows) >= 20
    half = len(rows) // 2
    for (n0, c0, t0, *_), (n1, c1, t1, *_) in zip(rows[:half], rows[half:]):
        assert n1 == n0 + ",merge" and (c0, t0) == (c1, t1)
    for name, chunks, threads, vgprs, scratch, lds, blocks in rows:
        assert threads in (256, 512, 1024) and 0 < vgprs <= 512 and lds > 0 and blocks >= 1
        assert name.startswith(f"fsamp_kernel<{threads},{chunks},")
    # the instantiations the benchmark configurations launch exist and keep every register in
    # VGPRs (no scratch); C5's tiling holds one 512-thread workgroup per CU
    by_name = {r[0]: r for r in rows}
    x = torch.zeros(256, 151936, dtype=torch.bfloat16, device="cuda")
    for b, v, k in ((1, 151936, 50), (8, 151936, 50), (16, 151936, 256), (16, 151936, 1024),
                    (256, 151936, 50), (1, 128256, 20), (4, 128256, 50), (16, 128256, 50),
                    (64, 128256, 50)):
        pl = fused_sampling.make_plan(x[:b, :v], k)
        name = f"fsamp_kernel<{pl.threads},{pl.chunks},vec>"
        if k > 128 and pl.splits > 1:
            name += ",merge"
        assert name in by_name, (b, v, k, name)
        assert by_name[name][4] == 0, f"{name} (B={b}, V={v}, k={k}) spills to scratch"
    c5 = by_name["fsamp_kernel<512,38,vec>"]
    assert c5[6] == 1 and c5[3] <= 256


def test_wave_primitives_have_the_lane_layouts_the_kernel_assumes():
    # DPP / swizzle / bpermute moves, the bitonic network and the fixed-order scan
    out = torch.zeros(12 * 64, dtype=torch.int32, device="cuda")
    import ctypes
    _lib.check(_lib.load().fsamp_debug_wave_selftest(ctypes.c_void_p(out.data_ptr()), None))
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).reshape(12, 64)
    lanes = np.arange(64, dtype=np.uint32)
    for r, j in enumerate((1, 2, 4, 8, 16, 32)):
        assert np.array_equal(got[r], lanes ^ j), f"xor_lane<{j}>"
    assert np.array_equal(got[6], 63 - lanes), "wave sort of a permutation"
    assert np.array_equal(got[7].view(np.float32), ((lanes + 1) * (lanes + 2) / 2).astype(np.float32))
    assert np.array_equal(got[8].view(np.float32), lanes.astype(np.float32))
    assert np.array_equal(got[9].view(np.float32), (lanes + 1).astype(np.float32))
    hi = (lanes * 21) & 63
    order = np.argsort(-hi.astype(np.int64), kind="stable")
    assert np.array_equal(got[10], hi[order]) and np.array_equal(got[11], 0xFFFFFFFF - lanes[order])


# --- per-row top_k / top_p / temperature (fsamp_sample_ex) -------------------------------------

def _row_controls(B, K, seed):
    g = np.random.Generator(np.random.PCG64(seed))
    ks = g.integers(1, K + 1, B).astype(np.int32)
    ks[:4] = [1, K, 0, K + 7][:min(4, B)]  # clamped to [1, K]
    ps = g.uniform(0.05, 1.0, B).astype(np.float32)
    ps[4:8] = [1.0, 1.5, 0.0, 0.999][:max(0, min(4, B - 4))]
    ts = g.uniform(0.3, 3.0, B).astype(np.float32)
    ts[8:12] = [1.0, 0.0, -2.0, 0.05][:max(0, min(4, B - 8))]
    return ks, ps, ts


@pytest.mark.parametrize("B,V,K,dtype", [(16, 151936, 50, "bfloat16"),   # split rows
                                         (40, 32000, 100, "float16"),    # one workgroup per row
                                         (12, 151936, 1024, "bfloat16"),  # wide k, LDS tail
                                         (12, 20000, 300, "bfloat16")])  # k in (256, 512]
def test_per_row_controls_match_the_oracle_bit_for_bit(B, V, K, dtype):
    bits = randn_bits((B, V), 7000 + K, 3.0, dtype)
    x = dev(bits, dtype)
    un = ustream(B, 7100 + K)
    ks, ps, ts = _row_controls(B, K, 7200 + K)
    tok, keep, ren = fused_sampling.sample_fused_ex(
        x, K, 0.9, u=torch.from_numpy(un).cuda(), top_k_row=torch.from_numpy(ks).cuda(),
        top_p_row=torch.from_numpy(ps).cuda(), temperature=torch.from_numpy(ts).cuda(),
        stages=True)
    want = O.sample(bits, dtype, K, 0.9, un, return_stages=True, nthreads=8, top_k_row=ks,
                    top_p_row=ps, temperature=ts)
    assert np.array_equal(tok.cpu().numpy(), want.token_ids)
    assert np.array_equal(keep.cpu().numpy(), want.keep)
    assert np.array_equal(ren.cpu().numpy(), want.renormed)
    # and the plain entry agrees with the per-row entry when every row carries the call's values
    same = fused_sampling.sample_fused_ex(
        x, K, 0.9, u=torch.from_numpy(un).cuda(),
        top_k_row=torch.full((B,), K, dtype=torch.int32, device="cuda"),
        top_p_row=torch.full((B,), 0.9, dtype=torch.float32, device="cuda"),
        temperature=torch.ones(B, device="cuda"))
    assert torch.equal(same, fused.sample_fused_u(x, K, 0.9, torch.from_numpy(un).cuda()))


def test_greedy_temperature_returns_the_argmax_with_the_lowest_id_tie():
    bits = randn_bits((8, 5000), 7300, 2.0, "bfloat16")
    bits[:, 100] = bits[:, 17] = W.to_bits(np.float32([30.0]), "bfloat16")[0]
    x = dev(bits, "bfloat16")
    tok = fused_sampling.sample_fused_ex(x, 50, 0.9, u=torch.full((8,), 0.999, device="cuda"),
                                         temperature=torch.zeros(8, device="cuda"))
    assert (tok.cpu().numpy() == 17).all()


def test_per_row_controls_reject_wrong_arrays():
    x = dev(randn_bits((4, 1000), 7301, 2.0, "bfloat16"), "bfloat16")
    with pytest.raises(RuntimeError, match="top_k_row"):
        fused_sampling.sample_fused_ex(x, 50, 0.9, offset=0,
                                       top_k_row=torch.ones(4, dtype=torch.int64, device="cuda"))
    with pytest.raises(RuntimeError, match="temperature"):
        fused_sampling.sample_fused_ex(x, 50, 0.9, offset=0, temperature=torch.ones(3, device="cuda"))


# --- graph-safe generator draw -----------------------------------------------------------------

def _uniforms(seed, offset, B):
    return O.rng_uniform(seed, offset, B)


def test_eager_calls_and_graph_replays_draw_from_one_generator_stream():
    # The reference takes philox_cuda_state(4) from torch's default generator for every call,
    # eager or captured (csrc/fused_sampling.cu:441-447), and its test asserts that replays
    # advance the stream (tests/test_fused_kernel.py:273-285).  Here every eager call and every
    # replay must draw the uniforms splitmix64(seed, o, row) at the generator offset o it found,
    # and no two draws -- eager or replayed -- may share an offset.
    B = 16
    bits = randn_bits((B, 6000), 7400, 1.0, "bfloat16")  # flat enough that draws differ
    x = dev(bits, "bfloat16")
    gen = torch.cuda.default_generators[torch.cuda.current_device()]
    torch.manual_seed(2024)
    seed = gen.initial_seed()
    used = []

    def eager():
        o = gen.get_offset()
        tok = fused.sample_fused(x, 50, 0.95).cpu().numpy()
        assert gen.get_offset() == o + 4
        used.append(("eager", o, tok))

    eager()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fused.sample_fused(x, 50, 0.95)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    used.append(("warm-up", gen.get_offset() - 8, None))
    used.append(("warm-up", gen.get_offset() - 4, None))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fused.sample_fused(x, 50, 0.95)
    for _ in range(4):
        eager()
        o = gen.get_offset()
        g.replay()
        torch.cuda.synchronize()
        assert gen.get_offset() == o + 4, "a replay advances the generator by its 4"
        used.append(("replay", o, out.cpu().numpy()))
    eager()
    offsets = [o for _, o, _ in used]
    assert len(set(offsets)) == len(offsets), f"two draws shared an offset: {offsets}"
    for kind, o, tok in used:
        if tok is None:
            continue
        want = oracle(bits, "bfloat16", 50, 0.95, O.rng_uniform(seed, o, B)).token_ids
        assert np.array_equal(tok, want), (kind, o)
    replays = [t.tobytes() for k, _, t in used if k == "replay"]
    assert len(set(replays)) > 1, "replays draw fresh uniforms"


def test_graphs_captured_at_several_batch_sizes_replay_in_any_order():
    # graphs of split-row calls (splits forced) captured at B = 32, 8, 1 on the default capture
    # stream share the row counters; replaying them in another order must leave every one
    # correct (the per-call candidates never overlap the counters)
    V = 20000
    bits = randn_bits((32, V), 7600, 3.0, "bfloat16")
    x = dev(bits, "bfloat16")
    un = ustream(32, 7601)
    u = torch.from_numpy(un).cuda()
    want = {B: oracle(bits[:B], "bfloat16", 50, 0.9, un[:B]).token_ids for B in (32, 8, 1)}
    for B in (32, 8, 1):
        fused.sample_fused_u(x[:B], 50, 0.9, u[:B], 4)  # warm-up outside capture
    torch.cuda.synchronize()
    graphs, outs = {}, {}
    for B in (32, 8, 1):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs[B] = fused.sample_fused_u(x[:B], 50, 0.9, u[:B], 4)
        graphs[B] = g
    for B in (1, 8, 32, 8, 1, 1, 32):
        graphs[B].replay()
        torch.cuda.synchronize()
        assert np.array_equal(outs[B].cpu().numpy(), want[B]), B
        # eager calls of other sizes in between use the same counters
        e = fused.sample_fused_u(x[:3], 50, 0.9, u[:3], 4).cpu().numpy()
        assert np.array_equal(e, oracle(bits[:3], "bfloat16", 50, 0.9, un[:3]).token_ids)


def test_device_seed_and_offset_sources_follow_philox_unpack():
    # fsamp_run with seed_ptr / offset_ptr draws splitmix64(*seed_ptr, *offset_ptr + offset, b)
    B = 8
    bits = randn_bits((B, 9000), 7700, 1.0, "bfloat16")
    x = dev(bits, "bfloat16")
    sp = torch.tensor([987654321], dtype=torch.int64, device="cuda")
    op = torch.tensor([4000], dtype=torch.int64, device="cuda")
    for splits in (1, 3):
        got = cabi.run(x, 50, 0.95, seed=1, offset=12, seed_ptr=sp, offset_ptr=op, splits=splits)
        want = oracle(bits, "bfloat16", 50, 0.95, O.rng_uniform(987654321, 4012, B)).token_ids
        assert np.array_equal(got.cpu().numpy(), want)
        only_off = cabi.run(x, 50, 0.95, seed=55, offset=3, offset_ptr=op, splits=splits)
        want = oracle(bits, "bfloat16", 50, 0.95, O.rng_uniform(55, 4003, B)).token_ids
        assert np.array_equal(only_off.cpu().numpy(), want)


def test_the_device_offset_counter_of_the_c_entry_advances_once_per_call():
    import ctypes
    B, V = 64, 30000
    bits = randn_bits((B, V), 7500, 1.0, "bfloat16")
    x = dev(bits, "bfloat16")
    lib = _lib.load()
    ctr = torch.tensor([1000], dtype=torch.int64, device="cuda")
    rows = _lib.RowParams(None, None, None, ctr.data_ptr())
    for splits in (1, 3):
        for call in range(2):
            c0 = int(ctr.item())
            out = torch.empty(B, dtype=torch.int64, device="cuda")
            stream = cabi.stream_ptr()
            ws = cabi.classic_workspace(x, 50, splits)
            _lib.check(lib.fsamp_sample_ex(ctypes.c_void_p(x.data_ptr()), 1, B, V, 50, 0.9, None,
                                           77, 123456, ctypes.byref(rows),
                                           ctypes.c_void_p(out.data_ptr()), None, None,
                                           cabi.vp(ws), ws.numel(), splits,
                                           ctypes.c_void_p(stream)))
            torch.cuda.synchronize()
            assert int(ctr.item()) == c0 + 4
            want = oracle(bits, "bfloat16", 50, 0.9, _uniforms(77, c0, B)).token_ids
            assert np.array_equal(out.cpu().numpy(), want)
    # without a workspace the counter form is refused (it needs the grid counter)
    assert lib.fsamp_sample_ex(ctypes.c_void_p(x.data_ptr()), 1, B, V, 50, 0.9, None, 77, 0,
                               ctypes.byref(rows), ctypes.c_void_p(out.data_ptr()), None, None,
                               None, 0, 1, None) == 6


# --- vocabulary shards: per-shard candidate words, then the merge and draw ---------------------

def _shard_words(x, k, bounds):
    ws = [fused_sampling.topk_shard(x[:, lo:hi], k, lo) for lo, hi in bounds]
    return torch.stack(ws, dim=1).contiguous()  # [B, N, k]


def _check_shard_words(words, bits, dtype, k, bounds):
    w = words.cpu().numpy().view(np.uint64)
    keys = O.key16(bits)
    for n, (lo, hi) in enumerate(bounds):
        ids = (0xFFFFFFFF - (w[:, n] & 0xFFFFFFFF)).astype(np.int64)
        want = oracle(np.ascontiguousarray(bits[:, lo:hi]), dtype, k, 1.0,
                      np.zeros(bits.shape[0], np.float32)).topk_ids + lo
        assert np.array_equal(ids, want), n
        assert np.array_equal((w[:, n] >> 32).astype(np.uint32),
                              np.take_along_axis(keys, ids, axis=1)), n


@pytest.mark.parametrize("name", ["C1", "C5"])
def test_eight_vocabulary_shards_merge_to_the_whole_row(name):
    c = W.case(name)
    x = dev(c.logits, c.dtype)
    N = 8
    Vs = c.vocab // N
    bounds = [(i * Vs, (i + 1) * Vs) for i in range(N)]
    words = _shard_words(x, c.top_k, bounds)
    _check_shard_words(words, c.logits, c.dtype, c.top_k, bounds)
    code = _lib.DTYPE_BF16 if c.dtype == "bfloat16" else _lib.DTYPE_F16
    ids = fused_sampling.merge_sample(words, code, c.top_p, ids_only=True).cpu().numpy()
    assert np.array_equal(ids, FIX[f"{name}/topk_ids"])
    u = torch.from_numpy(c.u).cuda()
    tok, keep, ren = fused_sampling.merge_sample(words, code, c.top_p, u, stages=True)
    want = oracle(c.logits, c.dtype, c.top_k, c.top_p, c.u)
    assert np.array_equal(tok.cpu().numpy(), FIX[f"{name}/token_ids"])
    assert np.array_equal(keep.cpu().numpy(), want.keep)
    assert np.array_equal(ren.cpu().numpy().view(np.uint32), want.renormed.view(np.uint32))
    alone = fused_sampling.merge_sample(words, code, c.top_p, u).cpu().numpy()
    assert np.array_equal(alone, FIX[f"{name}/token_ids"])


@pytest.mark.parametrize("k", [1, 50, 300, 1024])
def test_uneven_shards_and_wide_merges(k):
    # unaligned shard widths and offsets take the element-load path; k = 1024 over 8 shards
    # (8192 words) folds the lists from global memory instead of LDS
    B, V = 4, 151936 if k == 1024 else 40001
    bits = randn_bits((B, V), 7800 + k, 2.0, "float16")
    x = dev(bits, "float16")
    cuts = [0, 4999, 10007, 20001, 26003, 30000, 33333, 36667, V] if k <= 300 else \
        [i * (V // 8) for i in range(8)] + [V]
    bounds = list(zip(cuts[:-1], cuts[1:]))
    words = _shard_words(x, k, bounds)
    _check_shard_words(words, bits, "float16", k, bounds)
    un = ustream(B, 7900 + k)
    want = oracle(bits, "float16", k, 0.9, un)
    ids = fused_sampling.merge_sample(words, _lib.DTYPE_F16, 0.9, ids_only=True).cpu().numpy()
    assert np.array_equal(ids, want.topk_ids)
    tok = fused_sampling.merge_sample(words, _lib.DTYPE_F16, 0.9, torch.from_numpy(un).cuda())
    assert np.array_equal(tok.cpu().numpy(), want.token_ids)
    seeded = fused_sampling.merge_sample(words, _lib.DTYPE_F16, 0.9, seed=5, offset=9)
    want_s = oracle(bits, "float16", k, 0.9, O.rng_uniform(5, 9, B)).token_ids
    assert np.array_equal(seeded.cpu().numpy(), want_s)


def test_shard_and_merge_argument_checks():
    x = torch.zeros(2, 64, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="top_k must be <="):
        fused_sampling.topk_shard(x, 65, 0)
    w = torch.zeros(2, 3, 4, dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="top_p must be in"):
        fused_sampling.merge_sample(w, _lib.DTYPE_BF16, 0.0)
    with pytest.raises(RuntimeError, match="contiguous int64"):
        fused_sampling.merge_sample(w.float(), _lib.DTYPE_BF16, 0.5)


# --- large batches: the streaming selection of the big register tilings --------------------------

def _streaming_rows(V, seed):
    """128 rows that drive the streaming selection through each of its branches: plain noise,
    a 64-value tie grid (candidates overflow the register sort: the general path), ascending
    values (every candidate lands in the last chunks, after the bound), equal values, and a few
    spikes placed in the first and in the last chunks of a row."""
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal((128, V)).astype(np.float32) * 3.0
    grid = np.linspace(-8, 8, 64, dtype=np.float32)
    x[16:32] = grid[g.integers(0, 64, (16, V))]
    x[32:40] = np.linspace(-4, 4, V, dtype=np.float32)[None, :]
    x[40:44] = 0.5
    x[44:52, :64] += 20.0
    x[52:60, -64:] += 20.0
    return x


@pytest.mark.parametrize("V", [151936, 128256])
@pytest.mark.parametrize("k", [1, 20, 50, 64, 65])
def test_large_batch_rows_through_the_streaming_selection(V, k):
    rows = _streaming_rows(V, 8100 + k)
    if V == 128256:  # 256 rows: the streaming tiling (a grid of <= 192 takes 1024 x 16)
        rows = np.concatenate([rows, _streaming_rows(V, 9100 + k)])
    bits = W.to_bits(rows, "bfloat16")
    x = dev(bits, "bfloat16")
    pl = fused_sampling.make_plan(x, k)
    assert pl.splits == 1 and pl.threads == 512
    un = ustream(bits.shape[0], 8200 + k)
    want = oracle(bits, "bfloat16", k, 0.9, un)
    assert np.array_equal(fused.topk_fused(x, k).cpu().numpy(), want.topk_ids)
    tok, ids, keep, ren = run_u(x, k, 0.9, un)
    assert np.array_equal(tok, want.token_ids)
    assert np.array_equal(keep, want.keep)
    assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32))


def _tied_top_rows(V, seed):
    """128 rows of N(0, 1) noise with T equal top values (+20) spread over each row, T from 100
    to 320: the streaming selection's bound lands on the tied value, so a row has about T
    candidates (more where few of the ties fall in the prefix), across the register sorts'
    limits of 128 and 256 candidates."""
    g = np.random.Generator(np.random.PCG64(seed))
    x = g.standard_normal((128, V)).astype(np.float32)
    for r in range(128):
        t = 100 + (r * 220) // 127
        pos = np.linspace(0, V - 1, t).astype(np.int64) + g.integers(0, V // t, t) // 2
        x[r, np.minimum(pos, V - 1)] = 20.0
    return x


@pytest.mark.parametrize("V", [151936, 128256])
@pytest.mark.parametrize("k", [20, 50, 64])
def test_streaming_rows_with_129_to_256_candidates_sort_in_registers(V, k):
    rows = _tied_top_rows(V, 8400 + k)
    if V == 128256:  # 256 rows: the streaming tiling (a grid of <= 192 takes 1024 x 16)
        rows = np.concatenate([rows, _tied_top_rows(V, 9400 + k)])
    bits = W.to_bits(rows, "bfloat16")
    x = dev(bits, "bfloat16")
    pl = fused_sampling.make_plan(x, k)
    assert pl.splits == 1 and pl.threads == 512
    counts = fused_sampling.probe_phase(x, k, 0.9, 3, 0).cpu().numpy()
    # the rows span all three cases: the 128-candidate sort, the 256-candidate one, the re-read
    hist = ((counts <= 128).sum(), ((counts > 128) & (counts <= 256)).sum(), (counts > 256).sum())
    assert hist[0] >= 1 and hist[1] >= 40 and hist[2] >= 8, hist
    un = ustream(bits.shape[0], 8500 + k)
    want = oracle(bits, "bfloat16", k, 0.9, un)
    assert np.array_equal(fused.topk_fused(x, k).cpu().numpy(), want.topk_ids)
    tok, ids, keep, ren = run_u(x, k, 0.9, un)
    assert np.array_equal(tok, want.token_ids)
    assert np.array_equal(keep, want.keep)
    assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32))


@pytest.mark.parametrize("k", [57, 64])
def test_the_prefix_bound_keeps_noise_rows_within_the_register_sorts_up_to_k64(k):
    # with as many published thread maxima as k the bound would be the smallest of them and
    # noise rows would pass 256 candidates (the slice re-read); with the slack kept, none do
    bits = randn_bits((128, 151936), 8600 + k, 3.0, "bfloat16")
    x = dev(bits, "bfloat16")
    assert fused_sampling.make_plan(x, k).splits == 1
    counts = fused_sampling.probe_phase(x, k, 0.9, 3, 0).cpu().numpy()
    assert counts.min() >= k and counts.max() <= 256, (counts.min(), counts.max())
    un = ustream(128, 8700 + k)
    want = oracle(bits, "bfloat16", k, 0.9, un)
    tok, ids, keep, ren = run_u(x, k, 0.9, un)
    assert np.array_equal(tok, want.token_ids)


@pytest.mark.parametrize("k", [1, 50, 64, 100])
def test_32_chunk_rows_on_small_grids_take_1024_thread_workgroups(k):
    # V = 128256 in one slice at B <= 192: the planner's 1024 x 16 tiling (non-streaming)
    rows = _streaming_rows(128256, 8800 + k)
    bits = W.to_bits(rows, "bfloat16")
    x = dev(bits, "bfloat16")
    pl = fused_sampling.make_plan(x, k)
    assert pl.splits == 1 and pl.threads == 1024 and pl.chunks == 16
    un = ustream(128, 8900 + k)
    want = oracle(bits, "bfloat16", k, 0.9, un)
    assert np.array_equal(fused.topk_fused(x, k).cpu().numpy(), want.topk_ids)
    tok, ids, keep, ren = run_u(x, k, 0.9, un)
    assert np.array_equal(tok, want.token_ids)
    assert np.array_equal(keep, want.keep)
    assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32))


def test_sixteen_split_hand_off_at_b256():
    # the most workgroups per row (16) on the largest batch: 4096 workgroups whose row
    # tickets and candidate lists must hand over exactly once per row
    bits = randn_bits((256, 20000), 8300, 3.0, "bfloat16")
    x = dev(bits, "bfloat16")
    assert fused_sampling.make_plan(x, 50, 16).splits == 16
    un = ustream(256, 8301)
    want = oracle(bits, "bfloat16", 50, 0.9, un)
    tok, tok_stages, keep, ren = run_u(x, 50, 0.9, un, 16)
    assert np.array_equal(tok_stages, tok)
    assert np.array_equal(fused.topk_fused(x, 50, 16).cpu().numpy(), want.topk_ids)
    assert np.array_equal(tok, want.token_ids)
    assert np.array_equal(ren.view(np.uint32), want.renormed.view(np.uint32))
