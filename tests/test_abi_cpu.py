"""CPU checks of the C-ABI library: it loads, exports every entry point that
include/wh_sample.h declares, its structs match the ctypes mirror, and
host-side argument validation rejects what the reference rejects -- all
without touching a GPU (invalid calls return before any HIP call)."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wh_sample.h")


@pytest.fixture(scope="module")
def L():
    from whallm_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from whallm_amd import build

        build.build()
    return _lib


def declared_functions():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\*?\s+\*?(wh_\w+)\s*\(", src, re.M)))


def test_library_exports_every_declared_symbol(L):
    names = declared_functions()
    assert len(names) >= 8
    lib = L.lib()
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (wh_\w+)", out))
    assert set(names) <= exported


def test_struct_layouts_match_ctypes(L, tmp_path):
    """Every field's offset and both structs' sizes, from gcc on the header,
    against the ctypes mirror."""
    lines = []
    for cname, cls in (("wh_sample_args", L.SampleArgs), ("wh_verify_args", L.VerifyArgs), ("wh_markov_args", L.MarkovArgs),
                      ("wh_top_logprobs_args", L.TopLogprobsArgs),
                      ("wh_history_args", L.HistoryArgs),
                      ("wh_lmhead_args", L.LmHeadArgs)):
        lines.append(f'printf("%zu\\n", sizeof({cname}));')
        for f in cls._fields_:
            lines.append(f'printf("%zu\\n", offsetof({cname}, {f[0]}));')
    prog = tmp_path / "layout.c"
    prog.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "wh_sample.h"\nint main(void){'
                    + "".join(lines) + "return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(prog), "-o", str(exe)], check=True)
    got = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True).stdout.split()))
    want = []
    for cls in (L.SampleArgs, L.VerifyArgs, L.MarkovArgs, L.TopLogprobsArgs, L.HistoryArgs, L.LmHeadArgs):
        want.append(ctypes.sizeof(cls))
        want += [getattr(cls, f[0]).offset for f in cls._fields_]
    assert got == want


def _args(L, **kw):
    a = L.SampleArgs()
    a.logits = 1 << 20  # never dereferenced: validation fails first
    a.dtype = L.DTYPE_F32
    a.B = 1
    a.V = 100
    a.row_stride = 100
    a.temperature = 1.0
    a.top_p = 1.0
    a.chain = L.CHAIN_MLX
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,needle", [
    (dict(dtype=7), "dtype"),
    (dict(V=0), "V must be"),
    (dict(V=300000, row_stride=300000), "V must be"),
    (dict(row_stride=50), "row_stride"),
    (dict(min_p=1.5), "min_p"),
    (dict(temperature=-1.0), "temperature"),
    (dict(top_k=100), "top_k"),                      # chain mlx: k must be < V (mlx_lm apply_top_k)
    (dict(repetition_penalty=-1.0), "penalty"),
    (dict(chain=5), "chain"),
    (dict(out_mode=3), "out_mode"),
])
def test_host_validation_rejects_bad_arguments(L, kw, needle):
    a = _args(L, **kw)
    rc = L.lib().wh_sample(ctypes.byref(a), None)
    assert rc in (L.WH_EINVAL, L.WH_ELIMIT)
    assert needle in L.lib().wh_last_error().decode()


def test_penalty_window_limit(L):
    a = _args(L, presence_penalty=0.5, history=1 << 20, history_len=1 << 20, history_stride=8192, presence_context=0)
    assert L.lib().wh_sample(ctypes.byref(a), None) == L.WH_ELIMIT
    assert "WH_MAX_WINDOW" in L.lib().wh_last_error().decode()


def test_verify_validation(L):
    a = L.VerifyArgs()
    a.B, a.n, a.V = 1, 2, 0
    assert L.lib().wh_verify_logprobs(ctypes.byref(a), None) == L.WH_ELIMIT
    a.V = 10
    a.temperature = 1.0
    a.target = 1 << 20
    a.accepted = 1 << 20
    a.token = 1 << 20
    a.draft_tokens = 1 << 20
    assert L.lib().wh_verify_logprobs(ctypes.byref(a), None) == L.WH_EINVAL  # draft rows missing at T > 0
    assert L.lib().wh_verify_fused(ctypes.byref(a), None) == L.WH_EINVAL


def test_python_mirror_validation_without_gpu():
    from whallm_amd import sample_utils as su

    with pytest.raises(ValueError):
        su.make_sampler(temp=1.0, min_p=2.0)
    with pytest.raises(ValueError):
        su.make_repetition_penalty(-0.5)
    with pytest.raises(NotImplementedError):
        su.make_logits_processors(logit_bias={1: 2.0})
    procs = su.make_logits_processors(repetition_penalty=1.1, presence_penalty=0.5, frequency_penalty=0.2)
    assert [p.kind for p in procs] == ["repetition", "presence", "frequency"]
    assert su.make_logits_processors() == []


def test_noalloc_limit_is_checked_before_any_gpu_call(L):
    # 4096 rows of V = 151,936 need far more than the no-allocation
    # entry point's scratch: rejected with WH_ELIMIT before any HIP call
    a = _args(L, B=4096, V=151936, row_stride=151936, uniforms=1 << 20, tokens=1 << 20)
    assert L.lib().wh_sample_noalloc(ctypes.byref(a), None) == L.WH_ELIMIT
    assert "WH_NOALLOC_SCRATCH_BYTES" in L.lib().wh_last_error().decode()
    assert L.lib().wh_sample_workspace_bytes(4096, 151936) > L.NOALLOC_SCRATCH_BYTES
    assert L.lib().wh_sample_workspace_bytes(64, 151936) <= L.NOALLOC_SCRATCH_BYTES


@pytest.mark.parametrize("kw,needle", [
    (dict(keep=20, m=10, capacity=25), "capacity"),
    (dict(keep=5000, capacity=8192, history_stride=8192), "keep"),
    (dict(history_stride=10), "history_stride"),
    (dict(capacity=0), "capacity"),
    (dict(m=-1), "m must"),
])
def test_history_append_validation(L, kw, needle):
    a = L.HistoryArgs()
    a.history, a.history_len, a.tokens = 1 << 20, 1 << 20, 1 << 20
    a.B, a.capacity, a.history_stride, a.keep, a.m = 2, 64, 64, 20, 1
    for k, v in kw.items():
        setattr(a, k, v)
    rc = L.lib().wh_history_append(ctypes.byref(a), None)
    assert rc in (L.WH_EINVAL, L.WH_ELIMIT)
    assert needle in L.lib().wh_last_error().decode()


def test_top_logprobs_validation(L):
    a = L.TopLogprobsArgs()
    a.logits, a.top_ids, a.top_logprobs = 1 << 20, 1 << 20, 1 << 20
    a.B, a.V, a.n, a.row_stride = 2, 100, 65, 100
    assert L.lib().wh_top_logprobs(ctypes.byref(a), None) == L.WH_ELIMIT
    a.n = 5
    assert L.lib().wh_top_logprobs(ctypes.byref(a), None) == L.WH_EINVAL  # no workspace
    assert "workspace" in L.lib().wh_last_error().decode()
    assert L.lib().wh_top_logprobs_workspace_bytes(2, 100, 5) == 2 * 16 + 2 * 5 * 8


def test_decode_state_host_checks():
    from whallm_amd.decode import DecodeState, TokenSelector

    with pytest.raises(ValueError):
        DecodeState(2, 20, 20, "cpu")
    sel = TokenSelector(temperature=0.7, repetition_penalty=1.2, repetition_context=32, presence_penalty=0.5,
                        presence_context=8)
    assert sel.window == 32 and sel.penalised
    assert TokenSelector(presence_penalty=0.5, presence_context=0).window is None
    assert not TokenSelector(repetition_penalty=1.0).penalised


def test_lmhead_validation(L):
    a = L.LmHeadArgs()
    a.x, a.weight, a.logits_out, a.tokens = 1 << 20, 1 << 20, 1 << 20, 1 << 20
    a.M, a.K, a.V, a.logits_stride = 4, 512, 1000, 1000
    for kw, code, needle in ((dict(M=65), L.WH_ELIMIT, "M must"), (dict(K=100), L.WH_EINVAL, "K must"),
                             (dict(V=0), L.WH_ELIMIT, "V must"), (dict(x=(1 << 20) + 8), L.WH_EINVAL, "aligned"),
                             (dict(logits_stride=999), L.WH_EINVAL, "logits_stride")):
        b = L.LmHeadArgs.from_buffer_copy(a)
        for k, v in kw.items():
            setattr(b, k, v)
        assert L.lib().wh_lmhead_logits(ctypes.byref(b), None) == code, kw
        assert needle in L.lib().wh_last_error().decode()
    # the greedy form needs its workspace
    assert L.lib().wh_lmhead_greedy(ctypes.byref(a), None) == L.WH_EINVAL
    assert "workspace" in L.lib().wh_last_error().decode()
    assert L.lib().wh_lmhead_greedy_workspace_bytes(4, 1000) == 4 * 8 * 8
    # the fused call validates both halves before any launch
    s = _args(L, B=4, V=1000, row_stride=1000, tokens=1 << 20, uniforms=None)
    assert L.lib().wh_lmhead_sample(ctypes.byref(a), ctypes.byref(s), None) == L.WH_EINVAL
    assert "uniforms" in L.lib().wh_last_error().decode()
    b = L.LmHeadArgs.from_buffer_copy(a)
    b.logits_out = None
    assert L.lib().wh_lmhead_sample(ctypes.byref(b), ctypes.byref(s), None) == L.WH_EINVAL


def test_markov_validation(L):
    a = L.MarkovArgs()
    a.base, a.embed, a.proj, a.prev, a.logits_out = 1 << 20, 1 << 20, 1 << 20, 1 << 20, 1 << 20
    a.dtype, a.V, a.rank = L.DTYPE_BF16, 1000, 256
    for kw, needle in ((dict(rank=12), "rank"), (dict(rank=264), "rank"), (dict(dtype=5), "dtype"),
                       (dict(proj=(1 << 20) + 2), "aligned"), (dict(prev=None), "NULL")):
        b = L.MarkovArgs.from_buffer_copy(a)
        for k, v in kw.items():
            setattr(b, k, v)
        assert L.lib().wh_markov_logits(ctypes.byref(b), None) in (L.WH_EINVAL, L.WH_ELIMIT), kw
        assert needle in L.lib().wh_last_error().decode()
