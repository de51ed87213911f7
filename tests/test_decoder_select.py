"""Host-side choice of the batch-1 decode path (no GPU): the persistent
step only where its one-pass attention covers the cache and the library
accepts the shape on the device (kuiops_decode_step_supported: shape gate
plus occupancy query); every refusal selects the per-op graph."""
import torch

from kuillm_amd.decoder import LlamaShape, persistent_step_ok

CONFIG5 = LlamaShape(vocab=32000, d=2048, ffn=5632, layers=16, hq=32, hkv=8)
HD128 = LlamaShape(vocab=512, d=512, ffn=1536, layers=3, hq=4, hkv=1)


def accept(*args):
    return True


def refuse(*args):
    return False


def test_persistent_when_library_accepts():
    calls = []

    def spy(*args):
        calls.append(args)
        return True

    assert persistent_step_ok(CONFIG5, 1, 640, torch.bfloat16, True, supported=spy)
    assert calls == [(16, 2048, 5632, 32, 8, 64, 32000, 640, torch.bfloat16)]


def test_refused_by_library_takes_per_op_step():
    # e.g. the occupancy query finds that a step work-group does not fit a CU
    assert not persistent_step_ok(CONFIG5, 1, 640, torch.bfloat16, True, supported=refuse)


def test_cache_beyond_one_pass_attention_takes_per_op_step():
    assert persistent_step_ok(CONFIG5, 1, 768, torch.bfloat16, True, supported=accept)
    assert not persistent_step_ok(CONFIG5, 1, 769, torch.bfloat16, True, supported=accept)
    assert persistent_step_ok(HD128, 1, 384, torch.bfloat16, True, supported=accept)
    assert not persistent_step_ok(HD128, 1, 385, torch.bfloat16, True, supported=accept)


def test_batches_and_unfused_shapes_never_persistent():
    assert not persistent_step_ok(CONFIG5, 2, 640, torch.bfloat16, True, supported=accept)
    assert not persistent_step_ok(CONFIG5, 1, 640, torch.bfloat16, False, supported=accept)
    big_vocab = LlamaShape(vocab=40000, d=2048, ffn=5632, layers=16, hq=32, hkv=8)
    assert not persistent_step_ok(big_vocab, 1, 640, torch.bfloat16, True, supported=accept)
