"""The wide exact engine (rows with top-p alone, or no filter) against the
oracle: tokens and kept counts bit-exact, rows within 1e-5 in probability.
Covers large nuclei (flat rows), quantised values with ties at the cut,
-inf entries and all -inf rows, per-row temperature / top-p arrays mixing
greedy and unfiltered rows, penalties, both row outputs, and a boundary bin
too large for the list (the row then runs the whole exact algorithm)."""
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu


def announce(msg):
    sys.stderr.write(f"[gpu-case] {msg}\n")
    sys.stderr.flush()


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from whallm_amd import _lib

    _lib.lib()
    return torch.device("cuda:0")


def _rows(rng, B, V, kind):
    if kind == "flat":
        x = rng.normal(0, 2.5, (B, V))
    elif kind == "peaky":
        x = rng.normal(0, 2.0, (B, V))
        for b in range(B):
            x[b, rng.integers(0, V, 30)] += 9.0
    elif kind == "quant":
        x = np.round(rng.normal(0, 2.0, (B, V)) / 0.125) * 0.125
    elif kind == "masked":
        x = rng.normal(0, 2.0, (B, V))
        x[rng.random((B, V)) < 0.5] = -np.inf
        x[0, :] = -np.inf
    return x.astype(np.float32)


def _check_rows(got, want):
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    g, w = got[fin].astype(np.float64), want[fin].astype(np.float64)
    assert np.allclose(np.exp(g), np.exp(w), rtol=1e-5, atol=1e-12)


CASES = [
    # (B, V, kind, chain, T, top_p, dtype)
    (1, 129280, "flat", 0, 0.2, 0.98, "f32"),
    (1, 129280, "peaky", 0, 0.7, 0.95, "f32"),
    (1, 151936, "flat", 1, 0.8, 0.9, "bf16"),
    (3, 129280, "flat", 0, 0.7, 1.0, "f32"),
    (5, 40000, "quant", 0, 1.0, 0.5, "f32"),
    (5, 40000, "quant", 1, 0.6, 0.8, "bf16"),
    (4, 20001, "masked", 0, 1.3, 0.9, "f32"),
    (17, 4097, "flat", 1, 1.0, 0.999, "f32"),
    (2, 262144, "flat", 0, 0.9, 0.98, "f32"),
    (64, 151936, "flat", 0, 1.0, 0.9, "bf16"),
    (12, 129280, "quant", 0, 0.9, 0.95, "f32"),
]


@pytest.mark.parametrize("B,V,kind,chain,T,top_p,dtype", CASES)
def test_wide_tokens_and_counts(dev, oracle, B, V, kind, chain, T, top_p, dtype):
    from whallm_amd import sampling
    from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits

    rng = np.random.default_rng(V + B + int(T * 10))
    x = _rows(rng, B, V, kind)
    if dtype == "bf16":
        bits = f32_to_bf16_bits(x)
        x = bf16_bits_to_f32(bits)
        xt = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(x).to(dev)
    u = rng.random(B, dtype=np.float32)
    u[0] = 0.0
    p = oracle.make_params(B, temperature=T, top_p=top_p, chain=chain)
    ot, ok = oracle.sample(x, p, u)
    announce(f"wide engine B={B} V={V} {kind} chain={chain} T={T} p={top_p} {dtype}")
    tok, kept = sampling.sample(xt, temperature=T, top_p=top_p, chain="mlx" if chain == 0 else "whallm",
                                uniforms=torch.from_numpy(u).to(dev), return_kept=True)
    paths = sampling.last_paths(dev, B).cpu().numpy()
    assert np.all(np.isin(paths, (6, 1))), paths
    assert np.array_equal(kept.cpu().numpy(), ok)
    assert np.array_equal(tok.cpu().numpy(), ot)


def test_wide_rows_per_row_params_and_penalties(dev, oracle):
    from whallm_amd import sampling

    rng = np.random.default_rng(77)
    B, V, H = 8, 50000, 300
    x = _rows(rng, B, V, "flat")
    T = np.array([0.0, 0.7, 1.0, 0.2, 1.5, 0.0, 0.9, 1.0])
    tp = np.array([0.9, 1.0, 0.95, 0.98, 0.5, 1.0, 0.999, 1.0])
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hlen = rng.integers(0, H + 1, B).astype(np.int32)
    pen = dict(repetition_penalty=1.2, presence_penalty=0.5, frequency_penalty=0.2, repetition_context=64,
               presence_context=0, frequency_context=100)
    u = rng.random(B, dtype=np.float32)
    for chain in (0, 1):
        p = oracle.make_params(B, temperature=T, top_p=tp, chain=chain, **pen)
        ot, ok, orow = oracle.sample(x, p, u, hist, hlen, want_rows=True)
        announce(f"wide engine per-row params chain={chain}")
        kw = dict(temperature=1.0, top_p=1.0, chain="mlx" if chain == 0 else "whallm",
                  history=torch.from_numpy(hist).to(dev), history_len=torch.from_numpy(hlen).to(dev),
                  temperature_rows=torch.from_numpy(T).to(dev), top_p_rows=torch.from_numpy(tp).to(dev),
                  uniforms=torch.from_numpy(u).to(dev), **pen)
        if chain == 1:
            tok, rows, kept = sampling.sample(torch.from_numpy(x).to(dev), return_logprobs=True, return_kept=True, **kw)
            _check_rows(rows.cpu().numpy(), orow)
        else:
            tok, kept = sampling.sample(torch.from_numpy(x).to(dev), return_kept=True, **kw)
        paths = sampling.last_paths(dev, B).cpu().numpy()
        assert set(paths.tolist()) <= {1, 2, 6}, paths
        assert np.array_equal(tok.cpu().numpy(), ot)
        k = kept.cpu().numpy()
        g = T > 0
        assert np.array_equal(k[g], ok[g])
    # masked rows (the kept entries, -inf elsewhere)
    p = oracle.make_params(B, temperature=T, top_p=tp, chain=0, **pen)
    announce("wide engine masked rows")
    out = sampling.filter_rows(torch.from_numpy(x).to(dev), chain="mlx", temperature=1.0, top_p=0.95,
                               out_mode=1, history=torch.from_numpy(hist).to(dev),
                               history_len=torch.from_numpy(hlen).to(dev), **pen).cpu().numpy()
    pm = oracle.make_params(B, temperature=1.0, top_p=0.95, chain=0, **pen)
    pen_x = oracle.penalize(x, pm, hist, hlen)
    _, okm = oracle.sample(x, pm, u, hist, hlen)
    for b in range(B):
        kept_b = np.isfinite(out[b])
        assert kept_b.sum() == okm[b]
        assert np.array_equal(out[b][kept_b], pen_x[b][kept_b])
        # the kept set is a prefix of (value desc, id desc)
        order = np.lexsort((-np.arange(V), -pen_x[b].astype(np.float64)))
        assert np.all(kept_b[order[:okm[b]]])


def test_wide_list_overflow_falls_back_exact(dev, oracle):
    """20,000 equal entries in the boundary bin exceed the 8,192-entry list:
    the row runs the whole exact algorithm and still matches."""
    from whallm_amd import sampling

    rng = np.random.default_rng(5)
    B, V = 2, 30000
    x = np.zeros((B, V), np.float32)
    x[:, :10000] = rng.normal(-5, 1, (B, 10000))
    u = np.array([0.3, 0.999], np.float32)
    p = oracle.make_params(B, temperature=0.8, top_p=0.5)
    ot, ok = oracle.sample(x, p, u)
    announce("wide engine list overflow")
    tok, kept = sampling.sample(torch.from_numpy(x).to(dev), temperature=0.8, top_p=0.5,
                                uniforms=torch.from_numpy(u).to(dev), return_kept=True)
    assert sampling.last_paths(dev, B).cpu().numpy().tolist() == [1, 1]
    assert np.array_equal(kept.cpu().numpy(), ok)
    assert np.array_equal(tok.cpu().numpy(), ot)


@pytest.mark.parametrize("tied,lead", [(3000, 100), (300, 20), (900, 0)])
def test_wide_boundary_sub_bins(dev, oracle, tied, lead):
    """Boundary lists above 64 entries go through 256 sub-bins of the
    boundary bin: `tied` equal values with the cut among them (more than
    1024 in one sub-bin takes the radix select), `lead` values above them,
    and values near the tied one in the same bin but other sub-bins."""
    from whallm_amd import sampling

    rng = np.random.default_rng(tied + lead)
    B, V = 3, 40000
    x = np.full((B, V), -40.0, np.float32)
    for b in range(B):
        ids = rng.permutation(V)
        x[b, ids[:lead]] = 5.0
        x[b, ids[lead:lead + tied]] = 2.0
        # neighbours inside the same 1/64-nat bin, in other sub-bins
        x[b, ids[lead + tied:lead + tied + 200]] = 2.0 - rng.uniform(0.0, 0.0155, 200).astype(np.float32)
    u = np.array([0.0, 0.5, 0.999], np.float32)
    mass_lead = lead * 1.0
    mass_tied = tied * np.exp(-3.0) if lead else tied * 1.0
    top_p = float((mass_lead + 0.5 * mass_tied) / (mass_lead + mass_tied + 200 * np.exp(-3.0)))
    for chain in (0, 1):
        p = oracle.make_params(B, temperature=0.7, top_p=top_p, chain=chain)
        ot, ok = oracle.sample(x, p, u)
        announce(f"wide engine sub-bins tied={tied} lead={lead} chain={chain} p={top_p:.4f}")
        tok, kept = sampling.sample(torch.from_numpy(x).to(dev), temperature=0.7, top_p=top_p,
                                    chain="mlx" if chain == 0 else "whallm", uniforms=torch.from_numpy(u).to(dev),
                                    return_kept=True)
        assert np.all(sampling.last_paths(dev, B).cpu().numpy() == 6)
        assert np.array_equal(kept.cpu().numpy(), ok)
        assert np.array_equal(tok.cpu().numpy(), ot)


@pytest.mark.parametrize("B,dtype", [(3, "f32"), (3, "bf16"), (12, "f32"), (12, "bf16")])
def test_wide_load_layouts_agree(dev, oracle, B, dtype):
    """Rows the vector loads read (V a multiple of 4, rows aligned to four
    entries) and the same rows as an offset view of a wider tensor (base and
    row stride off that alignment: the per-entry loads).  Tokens, kept
    counts and logprob rows equal the oracle's both ways, and the masked rows
    agree between the two."""
    from whallm_amd import sampling
    from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits

    V = 40000
    rng = np.random.default_rng(B * 31 + len(dtype))
    x = _rows(rng, B, V, "peaky")
    u = rng.random(B, dtype=np.float32)
    if dtype == "bf16":
        bits = f32_to_bf16_bits(x)
        x = bf16_bits_to_f32(bits)
        dense = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        dense = torch.from_numpy(x).to(dev)
    wide = torch.zeros(B, V + 3, device=dev, dtype=dense.dtype)
    wide[:, 1:V + 1] = dense
    view = wide[:, 1:V + 1]
    kw = dict(temperature=0.8, top_p=0.9)
    p = oracle.make_params(B, chain=1, **kw)
    ot, ok, orow = oracle.sample(x, p, u, want_rows=True)
    masked = []
    for name, xt in (("vector", dense), ("per-entry", view)):
        announce(f"wide engine load layout {name} B={B} {dtype}")
        tok, rows, kept = sampling.sample(xt, uniforms=torch.from_numpy(u).to(dev), return_logprobs=True,
                                          return_kept=True, chain="whallm", **kw)
        paths = sampling.last_paths(dev, B).cpu().numpy()
        assert np.all(np.isin(paths, (6, 1))), (name, paths)
        assert np.array_equal(kept.cpu().numpy(), ok), name
        assert np.array_equal(tok.cpu().numpy(), ot), name
        _check_rows(rows.cpu().numpy(), orow)
        masked.append(sampling.filter_rows(xt, chain="mlx", temperature=1.0, top_p=0.95, out_mode=1).cpu().numpy())
    assert np.array_equal(masked[0], masked[1])
    fin = np.isfinite(masked[0])
    assert np.array_equal(masked[0][fin], x[fin])


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_wide_penalties_long_slices(dev, oracle, dtype):
    """B > 8 (4096-entry slices; the histogram step's workgroups build one
    penalty table over four slices' ids): repetition, presence and frequency
    penalties over per-row histories, top-p alone, both chains; tokens and
    kept counts equal the oracle's."""
    from whallm_amd import sampling
    from whallm_amd.synth import bf16_bits_to_f32, f32_to_bf16_bits

    rng = np.random.default_rng(4242 + len(dtype))
    B, V, H = 12, 70000, 600
    x = _rows(rng, B, V, "peaky")
    hist = rng.integers(0, V, (B, H)).astype(np.int32)
    hist[:, :40] = np.argsort(-x, axis=1)[:, :40]  # penalise the rows' leaders too
    hlen = rng.integers(H // 2, H + 1, B).astype(np.int32)
    if dtype == "bf16":
        bits = f32_to_bf16_bits(x)
        x = bf16_bits_to_f32(bits)
        xt = torch.from_numpy(bits.view(np.int16)).to(dev).view(torch.bfloat16)
    else:
        xt = torch.from_numpy(x).to(dev)
    u = rng.random(B, dtype=np.float32)
    pen = dict(repetition_penalty=1.3, presence_penalty=0.6, frequency_penalty=0.3, repetition_context=0,
               presence_context=200, frequency_context=0)
    for chain, T, top_p in ((0, 0.2, 0.98), (1, 0.9, 0.9)):
        p = oracle.make_params(B, temperature=T, top_p=top_p, chain=chain, **pen)
        ot, ok = oracle.sample(x, p, u, hist, hlen)
        announce(f"wide engine penalties B={B} {dtype} chain={chain}")
        tok, kept = sampling.sample(xt, temperature=T, top_p=top_p, chain="mlx" if chain == 0 else "whallm",
                                    history=torch.from_numpy(hist).to(dev), history_len=torch.from_numpy(hlen).to(dev),
                                    uniforms=torch.from_numpy(u).to(dev), return_kept=True, **pen)
        paths = sampling.last_paths(dev, B).cpu().numpy()
        assert np.all(np.isin(paths, (6, 1))), paths
        assert np.array_equal(kept.cpu().numpy(), ok), chain
        assert np.array_equal(tok.cpu().numpy(), ot), chain
