"""GPU parity of the batched prompt (pio_qwen3_prefill): a prompt's positions
in one pass per layer -- every int8 linear once over all rows on the W8 MFMA
GEMM, causal attention and KV-cache rows for every position -- as the
reference forwards the whole prompt at its first step
(ip/models/qwen3_0_6b/architecture.py:204-213).

Bars, as for the step decoder (tests/test_gpu_decode.py): logits against the
float64 oracle (qwen3_ref.forward_all, evaluated in one batched pass) within
max(1e-4, 4x numpy-fp32's own error) of the logit rms, argmax agreement
wherever the oracle's top-2 gap is clear; fp16 KV as there. The decode steps
that follow a batched prompt read the cache it wrote, so their logits are held
to the same bar on the GPU's own ids."""
import sys

import numpy as np
import pytest

from oracle import qwen3_ref
from tests.test_gpu_decode import _assert_logit_bar, _check_argmax

pytestmark = pytest.mark.gpu


def _say(m):
    print(m, flush=True)
    sys.stdout.flush()


def _against_oracle(got, ids, pos, rcfg, w, what):
    seq = np.asarray(ids[:max(pos) + 1])
    e64 = qwen3_ref.forward_all(rcfg, w, seq, pos, np.float64)
    e32 = qwen3_ref.forward_all(rcfg, w, seq, pos, np.float32).astype(np.float64)
    errs, errs32 = [], []
    for i, p in enumerate(pos):
        rms = float(np.sqrt(np.mean(e64[i] * e64[i])))
        errs.append(float(np.abs(got[i] - e64[i]).max()) / rms)
        errs32.append(float(np.abs(e32[i] - e64[i]).max()) / rms)
        _say(f"{what}: position {p}: err {errs[-1]:.2e} (numpy fp32 {errs32[-1]:.2e})")
        _check_argmax(got[i:i + 1], e64[i:i + 1], 1e-3)
    _assert_logit_bar(errs, errs32, rcfg, what)


def _small(**over):
    from mod_amd.qwen3 import Qwen3Config
    kw = dict(n_layers=2, hidden=1024, n_heads=16, n_kv_heads=8, head_dim=128, intermediate=3072,
              vocab=1000, max_seq=256)
    kw.update(over)
    return Qwen3Config(**kw), qwen3_ref.Qwen3Config(**kw)


@pytest.mark.parametrize("kv_dtype", ["float32", "float16"])
def test_prefill_last_logits_and_chunks(torch_dev, kv_dtype):
    """A 70-token prompt in one batch: the last position's logits against the
    oracle; the same prompt in three batches (31 + 1 + 38 positions: the
    second starts from the first one's cache) gives the same logits to fp32
    rounding; and the next id is the argmax, as the step would write it."""
    from mod_amd.qwen3 import Qwen3Int8Decoder, random_weights
    cfg, rcfg = _small(kv_dtype=kv_dtype)
    w = random_weights(cfg, seed=61)
    dec = Qwen3Int8Decoder(cfg, w)
    P = 70
    prompt = np.random.default_rng(62).integers(0, cfg.vocab, size=P).astype(np.int32)
    dec.reset(prompt)
    dec.prefill(P, logits=True)
    ids, one = dec.read(P + 1, with_logits=True)
    assert np.array_equal(ids[:P], prompt)
    assert int(ids[P]) == int(np.argmax(one))
    _against_oracle(one[None], prompt, [P - 1], rcfg, w, f"prefill last logits ({kv_dtype} KV)")
    dec.reset(prompt)
    dec.prefill(31)
    dec.prefill(1)
    dec.prefill(P - 32, logits=True)
    _, three = dec.read(0, with_logits=True)
    rms = float(np.sqrt(np.mean(one.astype(np.float64) ** 2)))
    diff = float(np.abs(three - one).max()) / rms
    _say(f"one batch vs three: max diff {diff:.2e} x rms")
    assert diff <= (1e-4 if kv_dtype == "float32" else 2e-3), diff


def test_prefill_refuses_generated_positions(torch_dev):
    from mod_amd.ops import RocmError
    from mod_amd.qwen3 import Qwen3Int8Decoder, random_weights
    cfg, _ = _small(n_layers=1)
    dec = Qwen3Int8Decoder(cfg, random_weights(cfg, seed=63))
    dec.reset(np.arange(8, dtype=np.int32))
    with pytest.raises(RocmError, match="prompt positions"):
        dec.prefill(9)
    dec.prefill(8)
    with pytest.raises(RocmError, match="prompt positions"):
        dec.prefill(1)


@pytest.mark.parametrize("mode", ["persistent", "graph"])
def test_prefill_then_decode_small(torch_dev, mode):
    """Prompt in one batch, then greedy steps: the steps' logits (the first
    generated position and every 8th) against the oracle on the GPU's own ids,
    and the ids agree with a run that consumes the prompt step by step."""
    from mod_amd.qwen3 import Qwen3Int8Decoder, random_weights
    cfg, rcfg = _small()
    w = random_weights(cfg, seed=64)
    dec = Qwen3Int8Decoder(cfg, w)
    P, NG = 40, 33
    prompt = np.random.default_rng(65).integers(0, cfg.vocab, size=P).astype(np.int32)
    dec.reset(prompt)
    dec.prefill(P - 1)
    pos, got, done = [], [], 0
    for n in [1] + [8] * 4:
        dec.run(n, mode=mode)
        done += n
        pos.append(P - 2 + done)          # the position the chunk's last step ran
        got.append(dec.read(0, with_logits=True)[1].copy())
    ids = dec.read(P + NG)
    assert np.array_equal(ids[:P], prompt)
    _against_oracle(np.stack(got), ids, pos, rcfg, w, f"prefill + {mode} steps")
    stepwise = dec.generate(prompt, NG, mode=mode)
    match = float(np.mean(stepwise == ids))
    _say(f"batched vs stepwise prompt: token match {match:.2f}")
    assert match >= 0.9


@pytest.mark.parametrize("kv_dtype", ["float32", "float16"])
def test_prefill_c2_generation_vs_oracle(torch_dev, kv_dtype):
    """BASELINE config 2 with the prompt as one batch: 28 layers, vocab
    151936, the 128-token prompt through pio_qwen3_prefill (its last
    position's logits produce the first generated id), then 255 persistent
    steps. The last prompt position's logits and those after every 32nd
    generated token meet the decoder bar against the batched oracle on the
    GPU's own ids, and each read argmax is the id generated next."""
    from mod_amd.qwen3 import Qwen3Config, Qwen3Int8Decoder, random_weights
    P, NG = 128, 256
    cfg = Qwen3Config(max_seq=P + NG, kv_dtype=kv_dtype)
    rcfg = qwen3_ref.Qwen3Config(max_seq=P + NG, kv_dtype=kv_dtype)
    _say("C2 batched prompt: building weights")
    w = random_weights(cfg, seed=0)
    dec = Qwen3Int8Decoder(cfg, w)
    mode = "persistent" if dec.persistent_supported() else "graph"
    prompt = np.random.default_rng(1).integers(0, cfg.vocab, size=P).astype(np.int32)
    dec.reset(prompt)
    dec.prefill(P, logits=True)
    pos = [P - 1]
    logits = [dec.read(0, with_logits=True)[1].copy()]
    done = 1
    for n in [32] * 7 + [31]:
        dec.run(n, mode=mode)
        done += n
        pos.append(P - 2 + done)
        logits.append(dec.read(0, with_logits=True)[1].copy())
    assert done == NG
    ids = dec.read(P + NG)
    assert np.array_equal(ids[:P], prompt)
    for p, lg in zip(pos, logits):
        assert int(np.argmax(lg)) == int(ids[p + 1]), p
    _say("C2 batched prompt: oracle (batched, teacher forced)")
    _against_oracle(np.stack(logits), ids, pos, rcfg, w, f"C2 batched prompt ({kv_dtype} KV)")
