"""The load-time self-check on the device: small llama-, Qwen2- and
LFM2-shaped models pass with errors near the output halves' rounding, the
engine is left reset, and a planted fault in the attention's output (forced
from the host: one head zeroed after the kernel ran) fails the check, sets
the simplest kernel forms and raises."""
import pytest
import torch

from webgllm_amd import engine as E, lib as L, ops, self_check as S

pytestmark = pytest.mark.gpu

SHAPES = {
    "llama": E.ModelShape("t-llama", 512, 2, 8, 2, 64, 1024, 4096, "q4_k_rowgroup",
                          rope_theta=5e5),
    "qwen2": E.ModelShape("t-qwen2", 896, 2, 14, 2, 64, 1024, 4096, "nbits", eps=1e-6),
    "lfm2": E.ModelShape("t-lfm2", 512, 4, 8, 8, 64, 1024, 4096, "q4_0", qk_norm=True,
                         conv_layers=(0, 2)),
}


@pytest.mark.parametrize("name", sorted(SHAPES))
def test_self_check_passes(hip, name):
    w = E.Weights(SHAPES[name], seed=11)
    eng, err = S.checked_engine(w, 256)
    print(f"{name}: self-check error {err:.2e}")
    assert err < 2e-3, err
    assert eng.position == 0 and eng.probe is None
    # the engine still decodes after the check
    out = eng.forward([1, 2, 3])
    assert out.shape[0] == 3


def test_self_check_catches_a_wrong_attention(hip, monkeypatch):
    w = E.Weights(SHAPES["llama"], seed=12)
    hd = SHAPES["llama"].head_dim
    real_decode, real_prefill = ops.attn_decode, ops.attn_prefill

    def zero_head(out):
        out[:, hd:2 * hd].zero_()
        return out

    monkeypatch.setattr(E.ops, "attn_decode",
                        lambda *a, **k: zero_head(real_decode(*a, **k)))
    monkeypatch.setattr(E.ops, "attn_prefill",
                        lambda *a, **k: zero_head(real_prefill(*a, **k)))
    saved = {k: L.tuning_get(k) for k in S.PLAIN_TUNING}
    try:
        eng = E.Engine(w, 256)
        assert S.self_check(eng) > S.SELF_CHECK_MAX
        with pytest.raises(S.SelfCheckError, match="computes the model wrong"):
            S.checked_engine(w, 256)
        # the retry ran with the simplest forms
        assert all(L.tuning_get(k) == v for k, v in S.PLAIN_TUNING.items())
    finally:
        for k, v in saved.items():
            L.tuning_set(k, v)
