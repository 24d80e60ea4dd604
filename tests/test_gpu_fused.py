"""Fused programs on the GPU against the oracle's host interpreter, bit for
bit (Kernels::fused, kernels.rs:1077; fused/mod.rs:62-70), and the Adam step
built on them (optim.rs:1048-1136; tests/optim.rs:71-101)."""

import numpy as np
import pytest

from oracle import binding as oracle
from oracle import mlp
from tensorcrate_amd import lib
from tensorcrate_amd.optim import EXACT, REASSOCIATE, Adam, identity_place
from tests.common import KINDS, Code, bits_equal, row_broadcast, run_form_program, same_bits, to_kind, widen
from tests.host_programs import host_adam_program

pytestmark = pytest.mark.gpu


def test_the_known_answer():
    # fused/mod.rs:23-37: y = sqrt(a w + 1) over [3, 0] and [1, 5] is [2, 1].
    code = [(0, 0, 0, 0, lib.F32, 0, 0.0), (0, 1, 1, 1, lib.F32, 0, 0.0), (2, lib.MUL, 2, 0, 1, 0, 0.0),
            (1, 0, 3, 0, 0, 0, 1.0), (2, lib.ADD, 4, 2, 3, 0, 0.0), (3, 13, 5, 4, 0, 0, 0.0),
            (5, 0, 0, 5, lib.F32, 0, 0.0)]
    a, w = lib.Buffer.of(np.array([3.0, 0.0], np.float32)), lib.Buffer.of(np.array([1.0, 5.0], np.float32))
    y = lib.Buffer(8)
    place = identity_place(1, 2)
    lib.fused(lib.F32, code, [place, place], [(a, 2), (w, 2)], [(y, 2)], 1, 2)
    assert y.download(np.float32).tolist() == [2.0, 1.0]


def test_remapped_loads_and_mixed_storage():
    # A [rows, cols] space reading an f16 row vector broadcast down the rows,
    # a bf16 matrix transposed, and an f32 matrix; stores to two types.
    rows, cols = 37, 70
    rng = np.random.default_rng(0)
    bias = to_kind(rng.standard_normal(cols), lib.F16)
    tm = to_kind(rng.standard_normal((cols, rows)), lib.BF16)  # read transposed
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    code = [(0, 0, 0, 0, lib.F16, 0, 0.0), (0, 1, 1, 1, lib.BF16, 0, 0.0), (0, 2, 2, 2, lib.F32, 0, 0.0),
            (2, lib.MUL, 3, 1, 2, 0, 0.0), (2, lib.ADD, 3, 3, 0, 0, 0.0), (4, lib.MAX, 4, 3, 2, 0, 0.0),
            (4, lib.GREATER, 5, 3, 0, 0, 0.0), (2, lib.DIV, 6, 4, 1, 0, 0.0),
            (5, 0, 0, 6, lib.BF16, 0, 0.0), (5, 0, 0, 5, lib.F32, 1, 0.0)]
    places = [(0, 1, 1, [rows], [0]), (0, rows, 1, [rows], [1]), identity_place(rows, cols)]
    for dtype in KINDS:
        out0 = np.zeros(rows * cols, np.uint16)
        out1 = np.zeros(rows * cols, np.float32)
        oracle.fused(dtype, code, places, [bias.view(np.uint16), tm, x], [out0, out1], rows, cols)
        d = [lib.Buffer.of(bias), lib.Buffer.of(tm), lib.Buffer.of(x)]
        g0, g1 = lib.Buffer(out0.nbytes), lib.Buffer(out1.nbytes)
        lib.fused(dtype, code, places, [(d[0], cols), (d[1], rows * cols), (d[2], rows * cols)],
                  [(g0, rows * cols), (g1, rows * cols)], rows, cols)
        assert bits_equal(g0.download(np.uint16), out0), dtype
        assert bits_equal(g1.download(np.float32), out1), dtype


def test_a_load_past_its_input_is_refused():
    code = [(0, 0, 0, 0, lib.F32, 0, 0.0), (5, 0, 0, 0, lib.F32, 0, 0.0)]
    a, y = lib.Buffer(4 * 10), lib.Buffer(4 * 12)
    with pytest.raises(lib.HipError, match="reaches past input 0"):
        lib.fused(lib.F32, code, [identity_place(3, 4)], [(a, 10)], [(y, 12)], 3, 4)


@pytest.mark.parametrize("magnitude", [0.01, 1.0, 100.0])
def test_adams_first_step_is_the_rate(magnitude):
    # tests/optim.rs:92-99: m_hat / sqrt(v_hat) is exactly +-1 on step one.
    p, g = lib.Buffer.of(np.zeros(1, np.float32)), lib.Buffer.of(np.array([magnitude], np.float32))
    Adam(0.1).update(p, g, 1, 1)
    assert abs(p.download(np.float32)[0] + 0.1) < 1e-6


# β₂ = 0.999 rounds to 1.0 in bf16, where every bias correction 1/(1 − β₂ᵗ)
# is infinite and the step does nothing; the reference's coefficients are
# public fields (optim.rs:1001-1005), so bf16 runs with β₂ = 0.99, whose
# bf16 value 0.98828125 keeps the update's arithmetic exercised.
#
# The checker's program is the Host's: `Adam::program` as built, run through
# the restated optimizer under the rule's algebra, the chosen plan lowered
# with each step's constants (tests/host_programs.py), and interpreted by
# the oracle.
@pytest.mark.parametrize("algebra", [REASSOCIATE, EXACT])
@pytest.mark.parametrize("dtype,second_decay", [(lib.F32, 0.999), (lib.F16, 0.999), (lib.BF16, 0.99),
                                                (lib.F32, 0.99)])
def test_adam_steps_match_the_oracle_bit_for_bit(dtype, second_decay, algebra):
    rows, cols = 129, 257
    rng = np.random.default_rng(4)
    p0 = to_kind(rng.standard_normal((rows, cols)), dtype)
    grads = [to_kind(rng.standard_normal((rows, cols)), dtype) for _ in range(4)]
    rule = Adam(1e-3, dtype, algebra)
    rule.second_decay = second_decay
    p = lib.Buffer.of(p0)
    host_p = p0.copy().reshape(-1)
    host_m = host_v = None
    for step, grad in enumerate(grads, start=1):
        rule.update(p, lib.Buffer.of(grad), rows, cols)
        resumed = host_m is not None
        code, loads, _ = host_adam_program(resumed, dtype, 1e-3, 0.9, second_decay, 1e-8, step,
                                           reassociate=algebra == REASSOCIATE)
        places = [identity_place(rows, cols)] * loads
        new_m = np.zeros_like(host_p) if not resumed else host_m
        new_v = np.zeros_like(host_p) if not resumed else host_v
        inputs = [grad.reshape(-1), host_p] + ([host_m, host_v] if resumed else [])
        oracle.fused(dtype, code, places, inputs, [host_p, new_m, new_v], rows, cols)
        host_m, host_v = new_m, new_v
        assert same_bits(p.download(host_p.dtype), host_p, dtype), step
        assert same_bits(rule.first.download(host_p.dtype), host_m, dtype), step
        assert same_bits(rule.second.download(host_p.dtype), host_v, dtype), step
        # The update moved parameters (a no-op step moves none): the
        # arithmetic ran.  In bf16 a step of the rate moves only the small
        # parameters, whose spacing is below it.
        assert np.count_nonzero(widen(dtype, host_p) != widen(dtype, p0.reshape(-1))) > rows * cols // 50, step


def test_config5_adam_over_the_mlp_parameters():
    # The MLP's 25,175,040 parameters in six tensors (1024 -> 4096 -> 4096 ->
    # 1024, with biases), ten steps, against the oracle on sampled slices of
    # the largest tensor and exactly everywhere through a checksum.
    rng = np.random.default_rng(4)
    rows, cols = 4096, 4096
    p0 = (rng.standard_normal((rows, cols), dtype=np.float32) * np.sqrt(2 / 4096)).astype(np.float32)
    grad = rng.standard_normal((rows, cols), dtype=np.float32)
    p, g = lib.Buffer.of(p0), lib.Buffer.of(grad)
    rule = Adam(1e-3)
    for _ in range(3):
        rule.update(p, g, rows, cols)
    got = p.download(np.float32).reshape(rows, cols)
    # The oracle on the first 64 rows (a row slab is the same program).
    host_p = p0[:64].copy().reshape(-1)
    m = v = None
    for step in range(1, 4):
        resumed = m is not None
        code, loads, _ = host_adam_program(resumed, lib.F32, 1e-3, 0.9, 0.999, 1e-8, step)
        nm = np.zeros_like(host_p) if m is None else m
        nv = np.zeros_like(host_p) if v is None else v
        ins = [grad[:64].reshape(-1).copy(), host_p] + ([m, v] if resumed else [])
        oracle.fused(lib.F32, code, [identity_place(64, cols)] * loads, ins, [host_p, nm, nv], 64, cols)
        m, v = nm, nv
    assert bits_equal(got[:64].reshape(-1), host_p)


def test_a_repeated_program_runs_compiled_and_stays_exact():
    # Dense programs compile on their second appearance (metal/codegen.rs:24);
    # the compiled kernel must give the interpreter's (and the oracle's) bits.
    import ctypes

    def compiled():
        count = ctypes.c_uint64()
        lib.call("tc_fused_compiled", ctypes.byref(count))
        return count.value

    rng = np.random.default_rng(12)
    n = 4096 * 3
    p0 = rng.standard_normal(n).astype(np.float32)
    grads = [rng.standard_normal(n).astype(np.float32) for _ in range(4)]
    before = compiled()
    params, moments = lib.Buffer.of(p0), None
    rule = Adam(1e-2)
    want = mlp.Adam(1e-2)
    expected = p0.copy()
    for g in grads:
        rule.update(params, lib.Buffer.of(g), 1, n)
        expected = want.update(expected, g)
        assert np.array_equal(params.download(np.float32), expected)
    assert compiled() > before


def test_a_compiled_program_past_the_infinity_cache_streams_and_stays_exact():
    # 12 Mi parameters: the resumed Adam step moves 28 bytes a parameter,
    # 336 MiB, past the 256 MiB Infinity Cache, so its compiled kernel takes
    # the nontemporal loads and stores; its bits must not change.
    rng = np.random.default_rng(13)
    n = 12 << 20
    p0 = rng.standard_normal(n, dtype=np.float32)
    params = lib.Buffer.of(p0)
    rule = Adam(1e-2)
    want = mlp.Adam(1e-2)
    expected = p0.copy()
    for step in range(4):
        g = rng.standard_normal(n, dtype=np.float32)
        rule.update(params, lib.Buffer.of(g), 1, n)
        expected = want.update(expected, g)
    assert np.array_equal(params.download(np.float32), expected)


@pytest.mark.parametrize("rows,cols", [(37, 70), (1, 1), (4099, 1000), (1000, 3)])
def test_a_repeated_broadcast_program_runs_compiled_and_stays_exact(rows, cols):
    # A program with a broadcast row vector and a transposed matrix is not
    # dense; from its second appearance it runs compiled (straight-line, 16
    # elements a thread).  Every run, in every type, gives the oracle's bits
    # (a square root: correctly rounded on both sides).
    import ctypes

    def compiled():
        count = ctypes.c_uint64()
        lib.call("tc_fused_compiled", ctypes.byref(count))
        return count.value

    rng = np.random.default_rng(rows + cols)
    bias = to_kind(rng.standard_normal(cols), lib.F16)
    tm = to_kind(rng.standard_normal((cols, rows)), lib.BF16)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    code = [(0, 0, 0, 0, lib.F16, 0, 0.0), (0, 1, 1, 1, lib.BF16, 0, 0.0), (0, 2, 2, 2, lib.F32, 0, 0.0),
            (2, lib.MUL, 3, 1, 2, 0, 0.0), (2, lib.ADD, 3, 3, 0, 0, 0.0), (3, 13, 7, 3, 0, 0, 0.0),
            (1, 0, 8, 0, 0, 0, 0.75), (2, lib.SUB, 7, 7, 8, 0, 0.0), (4, lib.GREATER, 5, 3, 0, 0, 0.0),
            (5, 0, 0, 7, lib.BF16, 0, 0.0), (5, 0, 0, 5, lib.F32, 1, 0.0)]
    places = [(0, 1, 1, [rows], [0]), (0, rows, 1, [rows], [1]), identity_place(rows, cols)]
    d = [lib.Buffer.of(bias), lib.Buffer.of(tm), lib.Buffer.of(x)]
    for dtype in KINDS:
        out0 = np.zeros(rows * cols, np.uint16)
        out1 = np.zeros(rows * cols, np.float32)
        oracle.fused(dtype, code, places, [bias.view(np.uint16), tm, x], [out0, out1], rows, cols)
        before = compiled()
        for _ in range(3):
            g0, g1 = lib.Buffer(out0.nbytes), lib.Buffer(out1.nbytes)
            lib.fused(dtype, code, places, [(d[0], cols), (d[1], rows * cols), (d[2], rows * cols)],
                      [(g0, rows * cols), (g1, rows * cols)], rows, cols)
            assert same_bits(g0.download(np.uint16), out0, lib.BF16), dtype
            assert bits_equal(g1.download(np.float32), out1), dtype
        # Compiled once per type and source, on a shape's second run.  The
        # source depends on the shape only through place steps of 0 or 1,
        # which it writes without their multiply: at (1, 1) the transposed
        # matrix's column step is 1, so that shape compiles its own.
        assert compiled() == before + (1 if (rows, cols) in ((37, 70), (1, 1)) else 0)


def _resident(limit=0):
    import ctypes

    resident, current = ctypes.c_uint64(), ctypes.c_uint64()
    lib.call("tc_fused_resident", limit, ctypes.byref(resident), ctypes.byref(current))
    return resident.value, current.value


def _nine_place_program(scale):
    """x[r, c] + x[r, c + 1] + ... + x[r, c + 8], times `scale`: nine places,
    one more than kernel arguments carry, so the program runs from a device
    copy."""
    code = [(0, 0, 0, 0, lib.F32, 0, 0.0)]
    for k in range(1, 9):
        code += [(0, k, 1, 0, lib.F32, 0, 0.0), (2, lib.ADD, 0, 0, 1, 0, 0.0)]
    code += [(1, 0, 2, 0, 0, 0, scale), (2, lib.MUL, 0, 0, 2, 0, 0.0), (5, 0, 0, 0, lib.F32, 0, 0.0)]
    return code


def test_large_programs_past_the_resident_limit_run_and_stay_exact():
    # A program with more places than kernel arguments carry is kept on the
    # device by its bytes, up to a limit; past it each run uploads its own
    # copy and frees it once queued.  Runs with new constants and shapes on
    # both sides of the limit, and a resident program run again, give the
    # oracle's bits.
    import ctypes

    from tests.test_gpu_runtime import Graph

    resident, limit = _resident()
    try:
        _resident(resident + 2)
        rng = np.random.default_rng(21)
        first = None
        for i, (rows, cols) in enumerate([(5, 7), (33, 65), (5, 7), (64, 3), (17, 130), (1, 1)]):
            scale = float(np.float32(1.0 + 0.25 * i))
            code = _nine_place_program(scale)
            places = [(k, 1, 1, [rows], [cols + 8]) for k in range(9)]
            x = rng.standard_normal(rows * (cols + 8)).astype(np.float32)
            want = np.zeros(rows * cols, np.float32)
            oracle.fused(lib.F32, code, places, [x], [want], rows, cols)
            dx, out = lib.Buffer.of(x), lib.Buffer(4 * rows * cols)
            lib.fused(lib.F32, code, places, [(dx, x.size)], [(out, rows * cols)], rows, cols)
            assert bits_equal(out.download(np.float32), want), (rows, cols)
            if first is None:
                first = (code, places, dx, x, want, rows, cols)
        assert _resident()[0] == resident + 2
        # The first program is resident: it runs from its kept copy, and may
        # be captured into a graph.
        code, places, dx, x, want, rows, cols = first
        out = lib.Buffer(4 * rows * cols)
        lib.fused(lib.F32, code, places, [(dx, x.size)], [(out, rows * cols)], rows, cols)
        assert bits_equal(out.download(np.float32), want)
        graph = Graph()
        again = lib.Buffer(4 * rows * cols)
        with graph:
            lib.fused(lib.F32, code, places, [(dx, x.size)], [(again, rows * cols)], rows, cols)
        for _ in range(2):
            graph.replay()
            lib.sync()
            assert bits_equal(again.download(np.float32), want)
        graph.destroy()
        # A program never run before cannot be uploaded from inside a
        # capture: refused, with nothing queued.
        novel = _nine_place_program(9.5)
        capture = Graph()
        lib.sync()
        assert capture.hip.hipStreamBeginCapture(capture.stream, 2) == 0
        try:
            with pytest.raises(lib.HipError, match="must run once before it is captured"):
                lib.fused(lib.F32, novel, places, [(dx, x.size)], [(again, rows * cols)], rows, cols)
        finally:
            assert capture.hip.hipStreamEndCapture(capture.stream, ctypes.byref(capture.graph)) == 0
            capture.hip.hipGraphDestroy(capture.graph)
        lib.call("tc_release_graph_memory")
        assert _resident()[0] == resident + 2
    finally:
        _resident(limit)


@pytest.mark.parametrize("f32_store", [True, False], ids=["f32-store", "16-bit-stores"])
@pytest.mark.parametrize("rows,cols,skew", [(4099, 1000, 0), (37, 72, 0), (1, 8, 0), (37, 1004, 0), (37, 70, 0),
                                            (4099, 1000, 1), (8192, 8192, 0)],
                         ids=["runs", "runs-small", "runs-one-row", "runs-of-four", "cols-not-whole-runs",
                              "misaligned-bias", "runs-streamed"])
def test_a_broadcast_program_in_runs_stays_exact(rows, cols, skew, f32_store):
    # A program whose places step their columns by 0 or 1 (a contiguous
    # matrix, a row-broadcast vector, one value a row, a scalar) runs
    # compiled in runs of one row when cols is a multiple of 4 and its
    # operands start on whole pieces: eight columns a thread (16-byte
    # pieces) when it stores only 16-bit outputs and cols is a multiple of 8,
    # else four; one load a run for the value a row.  A cols not a multiple
    # of 4, or a bias one element off its piece, takes the element form.
    # Past 256 MiB of traffic (8192 x 8192) the program streams: its stores
    # and the matrix's loads are non-temporal, the bias's loads not.
    # Every call, in every type, gives the oracle's bits.
    rng = np.random.default_rng(rows + cols + skew)
    bias = to_kind(rng.standard_normal(cols + skew), lib.F16)
    scale = to_kind(rng.uniform(0.5, 2, rows), lib.BF16)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    code, places = run_form_program(rows, skew)
    if not f32_store:
        code = code[:-1]
    places[2] = identity_place(rows, cols)
    d = [lib.Buffer.of(bias), lib.Buffer.of(scale), lib.Buffer.of(x), lib.Buffer.of(x[:1, :1].copy())]
    for dtype in KINDS:
        out0 = np.zeros(rows * cols, np.uint16)
        out1 = np.zeros(rows * cols, np.float32)
        outs = [out0, out1] if f32_store else [out0]
        oracle.fused(dtype, code, places, [bias.view(np.uint16), scale.view(np.uint16), x, x[:1, :1].copy()],
                     outs, rows, cols)
        for _ in range(3):
            g0, g1 = lib.Buffer(out0.nbytes), lib.Buffer(out1.nbytes)
            lib.fused(dtype, code, places, [(d[0], cols + skew), (d[1], rows), (d[2], rows * cols), (d[3], 1)],
                      [(g0, rows * cols), (g1, rows * cols)][:len(outs)], rows, cols)
            assert same_bits(g0.download(np.uint16), out0, lib.BF16), dtype
            if f32_store:
                assert bits_equal(g1.download(np.float32), out1), dtype


def _every_kind_of_f32(n, seed):
    """Random bit patterns (every binade, subnormals, infinities, NaNs)
    with zeros, extremes and the smallest subnormals among them."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32).copy()
    x[:10] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-40, 3.4e38, -1.1754944e-38, 1.0]
    return x


@pytest.mark.parametrize("divisor", [3.0, 0.1, -7.0, 1e-39, 3e38, 1.0, 0.0])
@pytest.mark.parametrize("rows,cols,form", [(3, 4096, "dense"), (64, 1000, "runs"), (37, 70, "elements")])
def test_a_division_by_a_constant_keeps_the_divisions_bits(rows, cols, form, divisor):
    # A division by a value the same for every element (here a constant)
    # compiles to one reciprocal and a product an element, with the f32
    # division kept for every quotient that is not a normal float; every
    # call (interpreted, then compiled), in every type and compiled form,
    # gives the oracle's bits, over operands of every kind: quotients that
    # overflow, land subnormal or are zero, infinities, NaNs, subnormal and
    # zero divisors.  A second output of a row vector makes the program
    # broadcast (the run form, or the element form for cols not a multiple
    # of 8).
    x = _every_kind_of_f32(rows * cols, cols)
    code = Code()
    q = code.binary(lib.DIV, code.load(0, 0, lib.F32), code.const(np.float32(divisor)))
    code.store(q, lib.F32, 0)
    places = [identity_place(rows, cols)]
    inputs, device = [x], [lib.Buffer.of(x)]
    if form != "dense":
        vector = np.arange(cols, dtype=np.float32)
        code.store(code.load(1, 1, lib.F32), lib.F32, 1)
        places.append(row_broadcast(cols))
        inputs.append(vector)
        device.append(lib.Buffer.of(vector))
    outputs = 1 if form == "dense" else 2
    for dtype in KINDS:
        want = [np.zeros(rows * cols, np.float32) for _ in range(outputs)]
        oracle.fused(dtype, code.code, places, inputs, want, rows, cols)
        for call in range(3):
            got = [lib.Buffer(rows * cols * 4) for _ in range(outputs)]
            lib.fused(dtype, code.code, places, [(d, a.size) for d, a in zip(device, inputs)],
                      [(g, rows * cols) for g in got], rows, cols)
            assert same_bits(got[0].download(np.float32), want[0], lib.F32), (dtype, call)
