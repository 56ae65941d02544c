"""Sequence snapshots on the host: payload layout, the reference-layout
conversions (pure tensor reshapes, run here on CPU tensors) and the C ABI's
argument checks.  The copies themselves run on the GPU (test_gpu_snapshot.py).
"""

from __future__ import annotations

import ctypes

import torch

from router_ia import _native as nat
from router_ia.snapshot import SequenceSnapshot, full_model_layers, linear_model_layers


def test_payload_size_closed_form():
    # 30 DeltaNet layers x 2 MiB, 30 conv rings x 4 x 8192 bf16, 10 layers x 63 pages x 2 heads x (8 KiB K + 8 KiB V)
    lin = 30 * 32 * 128 * 128 * 4
    conv = 30 * 4 * 8192 * 2
    kv = 10 * 63 * 2 * 16 * 256 * 2
    want = lin + conv + 2 * kv  # every section already a multiple of 256
    assert SequenceSnapshot.nbytes(30, 32, 8192, 10, 2, 1000) == want == 85_524_480
    assert SequenceSnapshot.nbytes(30, 32, 8192, 10, 2, 0) == lin + conv
    # a 17-token sequence needs two pages
    assert SequenceSnapshot.nbytes(0, 32, 8192, 1, 2, 17) == 2 * 2 * 2 * 8192


def test_model_layer_maps_follow_the_3_to_1_pattern():
    assert linear_model_layers(30)[:7] == [0, 1, 2, 4, 5, 6, 8] and linear_model_layers(30)[-1] == 38
    assert full_model_layers(10) == [3, 7, 11, 15, 19, 23, 27, 31, 35, 39]
    assert sorted(linear_model_layers(30) + full_model_layers(10)) == list(range(40))


def _reference_state(tokens, seed, n_lin=3, n_full=1):
    g = torch.Generator().manual_seed(seed)
    lin_layers, full_layers = linear_model_layers(n_lin), full_model_layers(n_full)
    conv = {}
    for m in lin_layers:
        w = torch.randn((1, 8192, 4), generator=g).to(torch.bfloat16)
        if tokens < 4:  # inputs before the first token are the zero-initialised state
            w[..., : 4 - tokens] = 0
        conv[m] = w
    return {
        "linear_states": {m: torch.randn((1, 32, 128, 128), generator=g) * 0.02 for m in lin_layers},
        "linear_conv_states": conv,
        "full_keys": {m: torch.randn((1, 2, tokens, 256), generator=g).to(torch.bfloat16) for m in full_layers},
        "full_values": {m: torch.randn((1, 2, tokens, 256), generator=g).to(torch.bfloat16) for m in full_layers},
        "tokens_seen": tokens,
    }


def test_reference_layout_round_trip_on_cpu():
    for tokens in (2, 16, 45):
        ref = _reference_state(tokens, tokens)
        snap = SequenceSnapshot.from_reference(ref, num_linear_layers=3, num_full_layers=1, device="cpu")
        back = snap.to_reference()
        assert back["tokens_seen"] == tokens
        for key in ("linear_states", "linear_conv_states", "full_keys", "full_values"):
            assert back[key].keys() == ref[key].keys()
            for m in ref[key]:
                assert torch.equal(back[key][m], ref[key][m].to(back[key][m].dtype)), (key, m, tokens)
        # slots past the sequence in its last page are zero in the payload
        kt = snap._tiles("k")
        if tokens % 16:
            assert not kt[:, -1, :, :, :, tokens % 16:, :].any()


def test_conv_ring_slots_hold_token_mod_4():
    ref = _reference_state(7, 3)
    snap = SequenceSnapshot.from_reference(ref, num_linear_layers=3, num_full_layers=1, device="cpu")
    rings = snap.conv_rings()
    window = ref["linear_conv_states"][0][0]  # [8192, 4]: tokens 3, 4, 5, 6
    for m, tok in enumerate(range(3, 7)):
        assert torch.equal(rings[0, tok % 4], window[:, m])


def test_save_restore_host_validation():
    lib = nat.load()
    fake = ctypes.c_void_p(256)
    rc = lib.ria_seq_state_save(3, 3, 30, 32, fake, fake, 8192, 10, 2, 100, fake, fake, fake, 64, 100, fake,
                                1 << 30, None)
    assert rc == 1 and b"row" in lib.ria_last_error()
    rc = lib.ria_seq_state_save(0, 3, 30, 32, fake, fake, 8192, 10, 2, 100, fake, fake, fake, 64, 100, fake, 1000,
                                None)
    assert rc == 3 and b"payload" in lib.ria_last_error()
    rc = lib.ria_seq_state_restore(0, 3, 30, 32, fake, fake, 8192, 10, 2, 100, fake, fake, fake, 4, 100, fake,
                                   1 << 30, None)
    assert rc == 1 and b"exceed" in lib.ria_last_error()
