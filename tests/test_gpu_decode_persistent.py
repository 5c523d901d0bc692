"""GPU parity of the persistent decode loop (pio_qwen3_run with
PIO_DECODE_PERSISTENT): all steps of a call run in one kernel launch that
hands data between workgroups through tagged words instead of kernel launches.

Same bar as the step-kernel decoder (test_gpu_decode.py): teacher-forced logits
against the float64 oracle within max(1e-4, 4x numpy-fp32's own error) of the
logit rms, argmax agreement wherever the oracle's top-2 gap is clear. On top:
the persistent kernel must agree with the graph path to fp32 rounding, and a
sequence decoded in one launch must equal the same sequence decoded over
several launches bit for bit (same arithmetic, positions/tags carried over)."""
import sys

import numpy as np
import pytest

from oracle import qwen3_ref
from tests.test_gpu_decode import _check_logits

pytestmark = pytest.mark.gpu


def _say(m):
    print(m, flush=True)
    sys.stdout.flush()


def _cfgs(**over):
    """Qwen3-0.6B layer shape (the persistent kernel's), fewer layers / vocab."""
    from mod_amd.qwen3 import Qwen3Config
    kw = dict(n_layers=2, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072,
              vocab=1000, max_seq=192)
    kw.update(over)
    return Qwen3Config(**kw), qwen3_ref.Qwen3Config(**kw)


def _decoder(cfg, seed):
    from mod_amd.qwen3 import Qwen3Int8Decoder, random_weights
    w = random_weights(cfg, seed=seed)
    dec = Qwen3Int8Decoder(cfg, w)
    if not dec.persistent_supported():
        from mod_amd import ops
        pytest.fail(f"persistent mode unsupported: {ops.last_error()}")
    return dec, w


@pytest.mark.parametrize("kv_dtype", ["float32", "float16"])
def test_persistent_teacher_forced_small(torch_dev, kv_dtype):
    cfg, rcfg = _cfgs(kv_dtype=kv_dtype)
    dec, w = _decoder(cfg, seed=11)
    ids = np.random.default_rng(12).integers(0, cfg.vocab, size=72).astype(np.int32)
    _say("persistent small: teacher forced, one launch per position")
    got = dec.teacher_forced_logits(ids, mode="persistent")
    np32_worst = _check_logits(got, ids, rcfg, w, "persistent small teacher-forced")
    _say("persistent small: graph path on the same ids")
    ref = dec.teacher_forced_logits(ids, mode="graph")
    rms = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    diff = float(np.abs(got - ref).max()) / rms
    _say(f"persistent vs graph: max diff {diff:.2e} x rms")
    # fp16 KV: the two paths sum k and v in different orders, so fp16
    # rounding flips differ between them as between any two fp32 paths
    assert diff <= (1e-4 if kv_dtype == "float32" else max(1e-4, 8 * np32_worst)), diff


def test_persistent_one_launch_equals_many(torch_dev):
    cfg, rcfg = _cfgs()
    dec, w = _decoder(cfg, seed=21)
    prompt = np.random.default_rng(22).integers(0, cfg.vocab, size=9).astype(np.int32)
    n_new = 40
    _say("persistent: one launch")
    one = dec.generate(prompt, n_new, mode="persistent")
    _say("persistent: four launches")
    dec.reset(prompt)
    for n in (5, 3, 25, len(prompt) - 1 + n_new - 33):
        dec.run(n, mode="persistent")
    many = dec.read(len(prompt) + n_new)
    assert np.array_equal(one[:len(prompt)], prompt)
    assert np.array_equal(one, many), (one, many)
    # mixed: prompt through the graph path, generation persistent (shared cache)
    _say("graph prompt + persistent generation")
    dec.reset(prompt)
    dec.run(len(prompt) - 1, mode="graph")
    dec.run(n_new, mode="persistent")
    mixed = dec.read(len(prompt) + n_new)
    got = dec.teacher_forced_logits(one, mode="persistent")
    _check_logits(got[:16], one, rcfg, w, "persistent greedy (own tokens)")
    ref_ids, _ = qwen3_ref.greedy(rcfg, w, list(prompt), n_new)
    match = np.mean(np.array(ref_ids) == one)
    _say(f"greedy token match vs oracle {match:.2f}; mixed-mode match {np.mean(mixed == one):.2f}")
    assert match >= 0.9, match
    assert np.mean(mixed == one) >= 0.9


@pytest.mark.parametrize("mode", ["persistent", "graph"])
@pytest.mark.parametrize("kv_dtype", ["float32", "float16"])
def test_decode_at_max_context(torch_dev, kv_dtype, mode):
    """The persistent kernel's context limit (2048 positions: 8 splits x 4
    waves x 8 positions x 8 passes): a 2040-position prompt as one batch, then
    the positions up to 2047 one launch each, every wave's last pass and the
    last position slot in use; the graph path on the same sequence (its
    attention splits of 256 positions); logits against the oracle."""
    cfg, rcfg = _cfgs(max_seq=2048, kv_dtype=kv_dtype)
    dec, w = _decoder(cfg, seed=41)
    ids = np.random.default_rng(42).integers(0, cfg.vocab, size=2048).astype(np.int32)
    dec.reset(ids)
    npre = 2040
    _say(f"max context ({kv_dtype}, {mode}): batched prompt of {npre}")
    dec.prefill(npre)
    got = []
    for _ in range(len(ids) - 1 - npre):
        dec.run(1, mode=mode)
        got.append(dec.read(0, with_logits=True)[1].copy())
    _say("max context: batched oracle")
    want = list(range(npre, len(ids) - 1))
    e64 = qwen3_ref.forward_all(rcfg, w, ids[:-1], want, np.float64)
    e32 = qwen3_ref.forward_all(rcfg, w, ids[:-1], want, np.float32).astype(np.float64)
    for k, i in enumerate(want):
        rms = float(np.sqrt(np.mean(e64[k] * e64[k])))
        err = float(np.abs(got[k] - e64[k]).max()) / rms
        err32 = float(np.abs(e32[k] - e64[k]).max()) / rms
        _say(f"position {i}: err {err:.2e} (numpy fp32 {err32:.2e})")
        assert err <= max(1e-4, 4 * err32), (i, err, err32)


def test_persistent_refresh_after_weights_change(torch_dev):
    """The persistent mode decodes from its own copy of the int8 layer
    weights: after the caller rewrites one in place, the graph path (which
    reads the caller's buffers) sees the change and the persistent path does
    not until pio_qwen3_refresh_weights; then the two agree again."""
    cfg, _ = _cfgs()
    dec, w = _decoder(cfg, seed=51)
    ids = np.random.default_rng(52).integers(0, cfg.vocab, size=40).astype(np.int32)

    def logits(mode):
        dec.reset(ids)
        dec.run(len(ids) - 1, mode=mode)
        return dec.read(0, with_logits=True)[1].astype(np.float64)

    def rel(a, b):
        return float(np.abs(a - b).max() / np.sqrt(np.mean(b * b)))

    _say("refresh: before the change")
    before = logits("persistent")
    assert rel(before, logits("graph")) < 1e-4
    ptr = dec._layers_c[1].w_down
    buf = next(t for t in dec._keep if t.data_ptr() == ptr)
    new_down = np.random.default_rng(53).integers(-127, 127, size=w["layers"][1]["w_down"].shape,
                                                  dtype=np.int8)
    buf.load(new_down)
    _say("refresh: after the change, before the refresh")
    g = logits("graph")
    assert rel(g, before) > 1e-2                      # the change matters
    assert rel(logits("persistent"), before) < 1e-4   # the stale copy still decodes as before
    dec.refresh_weights()
    _say("refresh: after the refresh")
    assert rel(logits("persistent"), g) < 1e-4


def test_persistent_long_context(torch_dev):
    """Contexts past 384 positions read part of each split's keys straight from
    the cache instead of the prefetched registers."""
    cfg, rcfg = _cfgs(max_seq=640)
    dec, w = _decoder(cfg, seed=31)
    ids = np.random.default_rng(32).integers(0, cfg.vocab, size=600).astype(np.int32)
    dec.reset(ids)
    tail = 4
    _say("persistent long context: prompt")
    dec.run(len(ids) - 1 - tail, mode="persistent")
    got = []
    for _ in range(tail):
        dec.run(1, mode="persistent")
        got.append(dec.read(0, with_logits=True)[1].copy())
    _say("persistent long context: oracle")
    r64 = qwen3_ref.Qwen3Ref(rcfg, w, np.float64)
    r32 = qwen3_ref.Qwen3Ref(rcfg, w, np.float32)
    for i, t in enumerate(ids[:-1]):
        e64 = r64.step(int(t))
        e32 = r32.step(int(t)).astype(np.float64)
        k = i - (len(ids) - 1 - tail)
        if k < 0:
            continue
        rms = float(np.sqrt(np.mean(e64 * e64)))
        err = float(np.abs(got[k] - e64).max()) / rms
        err32 = float(np.abs(e32 - e64).max()) / rms
        _say(f"position {i}: err {err:.2e} (numpy fp32 {err32:.2e})")
        assert err <= max(1e-4, 4 * err32), (i, err, err32)


def test_persistent_lm_head_small_vocab_and_ties(torch_dev):
    """The lm phase deals the vocabulary rows over the 256 workgroups and their
    waves in 16-row MFMA groups. With vocab 200, 56 workgroups own no row at
    all (their key must not win): teacher-forced logits against the oracle.
    With every lm_head row and scale equal, every logit ties: greedy decode
    must pick id 0 (the reference argmax keeps the first maximum,
    tensor_ops.c:649-662) across lanes, waves and workgroups, in the
    persistent mode as in the graph mode."""
    from mod_amd.qwen3 import Qwen3Int8Decoder, random_weights
    cfg, rcfg = _cfgs(vocab=200)
    dec, w = _decoder(cfg, seed=61)
    ids = np.random.default_rng(62).integers(0, cfg.vocab, size=24).astype(np.int32)
    _say("lm small vocab: teacher forced")
    got = dec.teacher_forced_logits(ids, mode="persistent")
    _check_logits(got, ids, rcfg, w, "persistent vocab 200")

    cfg, _ = _cfgs(vocab=4096)
    w = random_weights(cfg, seed=63)
    w["lm_head"] = np.ascontiguousarray(np.broadcast_to(w["lm_head"][:1], w["lm_head"].shape))
    w["s_lm_head"] = np.full_like(w["s_lm_head"], w["s_lm_head"][0])
    dec = Qwen3Int8Decoder(cfg, w)
    prompt = np.random.default_rng(64).integers(0, cfg.vocab, size=6).astype(np.int32)
    for mode in ("persistent", "graph"):
        _say(f"lm ties: greedy, {mode}")
        out = dec.generate(prompt, 12, mode=mode)
        assert np.array_equal(out[:len(prompt)], prompt)
        assert np.all(out[len(prompt):] == 0), (mode, out)


def test_persistent_lm_head_tiny_final_norm(torch_dev):
    """The lm phase splits gamma * x into int8 parts under the scale
    S = 2^(E - 6) of its largest element (2^E > max |gamma * x|). A final norm
    of 2^-126 puts E near -122, where 2^(6 - E) is past the fp32 range: the
    parts are formed by exponent arithmetic, so they stay exact and the
    teacher-forced logits still meet the oracle's bar."""
    from mod_amd.qwen3 import Qwen3Int8Decoder, random_weights
    cfg, rcfg = _cfgs(vocab=300)
    w = random_weights(cfg, seed=65)
    w["final_norm"] = np.full_like(w["final_norm"], 2.0 ** -126)
    dec = Qwen3Int8Decoder(cfg, w)
    ids = np.random.default_rng(66).integers(0, cfg.vocab, size=12).astype(np.int32)
    _say("lm tiny final norm: teacher forced")
    got = dec.teacher_forced_logits(ids, mode="persistent")
    assert np.isfinite(got).all()
    _check_logits(got, ids, rcfg, w, "persistent, final norm 2^-126")


def test_persistent_c2_shape(torch_dev):
    """Full Qwen3-0.6B shape (28 layers, vocab 151936)."""
    cfg, rcfg = _cfgs(n_layers=28, vocab=151936, max_seq=384)
    _say("persistent C2: building weights")
    dec, w = _decoder(cfg, seed=41)
    ids = np.random.default_rng(42).integers(0, cfg.vocab, size=7).astype(np.int32)
    _say("persistent C2: teacher forced")
    got = dec.teacher_forced_logits(ids, mode="persistent")
    _check_logits(got, ids, rcfg, w, "persistent C2 teacher-forced")
    _say("persistent C2: greedy persistent vs graph")
    prompt = ids[:5]
    a = dec.generate(prompt, 48, mode="persistent")
    b = dec.generate(prompt, 48, mode="graph")
    match = float(np.mean(a == b))
    _say(f"persistent vs graph greedy token match {match:.2f}")
    assert match >= 0.9


def _check_against_batched_oracle(got, ids, pos, rcfg, w, what):
    """got[i] = GPU logits after position pos[i] of the id sequence `ids`
    (teacher forcing on the GPU's own tokens): the bar of _check_logits, with
    the oracle evaluated in one batched pass (float64, and numpy float32 for
    the fp32 error scale)."""
    from tests.test_gpu_decode import _check_argmax
    seq = ids[:max(pos) + 1]
    e64 = qwen3_ref.forward_all(rcfg, w, seq, pos, np.float64)
    e32 = qwen3_ref.forward_all(rcfg, w, seq, pos, np.float32).astype(np.float64)
    from tests.test_gpu_decode import _assert_logit_bar
    errs, errs32 = [], []
    for i, p in enumerate(pos):
        rms = float(np.sqrt(np.mean(e64[i] * e64[i])))
        errs.append(float(np.abs(got[i] - e64[i]).max()) / rms)
        errs32.append(float(np.abs(e32[i] - e64[i]).max()) / rms)
        _say(f"{what}: position {p}: err {errs[-1]:.2e} (numpy fp32 {errs32[-1]:.2e})")
        _check_argmax(got[i:i + 1], e64[i:i + 1], 1e-3)
    _assert_logit_bar(errs, errs32, rcfg, what)
    _say(f"{what}: worst logit err {max(errs):.2e} x rms")


@pytest.mark.parametrize("kv_dtype", ["float32", "float16"])
def test_persistent_c2_full_generation_vs_oracle(torch_dev, kv_dtype):
    """BASELINE config 2 end to end: 28 layers, vocab 151936, a 128-token
    prompt and 256 greedy tokens (KV to 384 positions). The generation runs in
    chunks (1, 7 x 32, 31 tokens) so the logits of the first generated token,
    of every 32nd after it and of the last are read; they must meet the
    teacher-forced bar against the oracle on the GPU's own ids, the GPU's
    argmax at each of them must be the id it then generated, and the chunked
    run must produce the same 384 ids as one launch."""
    from mod_amd.qwen3 import Qwen3Config, Qwen3Int8Decoder, random_weights
    P, NG = 128, 256
    cfg = Qwen3Config(max_seq=P + NG, kv_dtype=kv_dtype)
    rcfg = qwen3_ref.Qwen3Config(max_seq=P + NG, kv_dtype=kv_dtype)
    _say("C2 full generation: building weights")
    w = random_weights(cfg, seed=0)
    dec = Qwen3Int8Decoder(cfg, w)
    if not dec.persistent_supported():
        from mod_amd import ops
        pytest.fail(f"persistent mode unsupported: {ops.last_error()}")
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, size=P).astype(np.int32)
    _say("C2 full generation: chunked")
    dec.reset(prompt)
    dec.run(P - 1, mode="persistent")
    pos, logits, done = [], [], 0
    for n in [1] + [32] * 7 + [31]:
        dec.run(n, mode="persistent")
        done += n
        pos.append(P - 2 + done)          # the position the chunk's last step ran
        logits.append(dec.read(0, with_logits=True)[1].copy())
    assert done == NG
    ids = dec.read(P + NG)
    assert np.array_equal(ids[:P], prompt)
    for p, lg in zip(pos, logits):
        assert int(np.argmax(lg)) == int(ids[p + 1]), p
    _say("C2 full generation: one launch")
    dec.reset(prompt)
    dec.run(P - 1 + NG, mode="persistent")
    assert np.array_equal(dec.read(P + NG), ids)
    _say("C2 full generation: oracle (batched, teacher forced)")
    _check_against_batched_oracle(np.stack(logits), ids, pos, rcfg, w, f"C2 full generation ({kv_dtype} KV)")


def test_persistent_rejects_other_shapes(torch_dev):
    from mod_amd.ops import RocmError
    from mod_amd.qwen3 import Qwen3Config, Qwen3Int8Decoder, random_weights
    cfg = Qwen3Config(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128,
                      intermediate=512, vocab=1000, max_seq=64)
    dec = Qwen3Int8Decoder(cfg, random_weights(cfg, seed=5))
    assert not dec.persistent_supported()
    dec.reset(np.arange(4, dtype=np.int32))
    with pytest.raises(RocmError):
        dec.run(2, mode="persistent")
    dec.run(2, mode="graph")   # the step path still serves it


def test_persistent_rejects_more_layers_than_its_constants_hold(torch_dev):
    """The persistent kernel keeps every layer's per-wave scales in LDS, sized
    for 48 layers: a 49-layer model of the supported layer shape is refused
    with an error that says so, and the graph path still serves it."""
    from mod_amd import ops
    cfg, _ = _cfgs(n_layers=49, max_seq=64)
    from mod_amd.qwen3 import Qwen3Int8Decoder, random_weights
    dec = Qwen3Int8Decoder(cfg, random_weights(cfg, seed=6))
    assert not dec.persistent_supported()
    assert "layers <= 48" in ops.last_error()
    dec.reset(np.arange(4, dtype=np.int32))
    with pytest.raises(ops.RocmError):
        dec.run(2, mode="persistent")
    dec.run(2, mode="graph")


def test_persistent_launch_without_the_whole_grid_reruns_in_graph_mode(torch_dev, monkeypatch):
    """A persistent launch needs every workgroup resident at once; one that
    does not get them (forced from the host: PIO_LOOP_ARRIVE_TICKS=0 makes the
    kernel's co-residency wait fail at once, so every wave exits normally)
    computes nothing, later persistent launches skip too, and the next read
    re-runs those steps in graph mode: the ids agree with a normal persistent
    run (the graph path rounds differently in fp32, so greedy ids may part at
    a near-tie: at least 90% must match, as between the modes elsewhere)."""
    cfg, _ = _cfgs()
    dec, _ = _decoder(cfg, seed=51)
    prompt = np.random.default_rng(52).integers(0, cfg.vocab, size=6).astype(np.int32)
    n_new = 24
    _say("co-residency fallback: reference run")
    want = dec.generate(prompt, n_new, mode="persistent")
    assert dec.persistent_replays() == 0
    dec.reset(prompt)
    dec.run(len(prompt) - 1, mode="persistent")          # resident: runs
    monkeypatch.setenv("PIO_LOOP_ARRIVE_TICKS", "0")
    _say("co-residency fallback: two launches that cannot start")
    dec.run(10, mode="persistent")
    dec.run(n_new - 10, mode="persistent")
    monkeypatch.delenv("PIO_LOOP_ARRIVE_TICKS")
    got = dec.read(len(prompt) + n_new)
    assert dec.persistent_replays() == 1
    assert np.array_equal(got[:len(prompt)], prompt)
    assert np.mean(got == want) >= 0.9, (got, want)
    # a graph-mode run after a failed launch settles it first
    dec.reset(prompt)
    dec.run(len(prompt) - 1, mode="persistent")
    monkeypatch.setenv("PIO_LOOP_ARRIVE_TICKS", "0")
    dec.run(10, mode="persistent")
    monkeypatch.delenv("PIO_LOOP_ARRIVE_TICKS")
    dec.run(n_new - 10, mode="graph")
    got2 = dec.read(len(prompt) + n_new)
    assert dec.persistent_replays() == 2
    assert np.mean(got2 == want) >= 0.9


def test_persistent_traced_launch_stamps_every_phase(torch_dev):
    """The traced build (pio_qwen3_trace_next) computes the same tokens as the
    product kernel and stamps every phase boundary of the two traced steps on
    every workgroup, in order."""
    cfg, _ = _cfgs()
    dec, _ = _decoder(cfg, seed=71)
    prompt = np.random.default_rng(72).integers(0, cfg.vocab, size=5).astype(np.int32)
    # traced steps at positions 64, 65: every attention split has positions
    want = dec.generate(prompt, 80, mode="persistent")
    dec.reset(prompt)
    dec.run(len(prompt) - 1, mode="persistent")
    dec.trace_next(60)
    dec.run(80, mode="persistent")
    assert np.array_equal(dec.read(len(prompt) + 80), want)
    t = dec.phase_trace()                          # [2][256][L + 1][16] ns
    L = cfg.n_layers
    att = (np.arange(256) // 8) < 8
    main = [0, 1, 2, 3, 5, 6, 7, 8, 9, 10]
    for s in range(2):
        blk = t[s, :, :L, :]
        assert np.isfinite(blk[:, 1:, main]).all()                 # layer 0 has no P1 reduction
        assert np.isfinite(blk[att][:, :, [4, 12, 13]]).all()
        assert np.isnan(blk[~att][:, :, 4]).all()
        order = blk[:, 1:, main]
        assert (np.diff(order, axis=-1) >= 0).all()
        assert np.isfinite(t[s, :, L, :5]).all()
    assert np.nanmin(t[1]) > np.nanmax(t[0, :, :L, :11])
