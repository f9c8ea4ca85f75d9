"""GPU: the int8 snapshot store. Row copies are exact bytes (multi-run, more runs than one launch carries, bounds
refused on the host); a snapshot restored into a fresh state gives back the original int8 K/V and scales bit for
bit; and the resume-then-prefill flow serves a cached prefix and leaves the state exactly as prefilling the same
pieces in order would."""
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rand_state(st, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    st.q.copy_(torch.randint(-127, 128, st.q.shape, generator=g, device=DEV, dtype=torch.int8))
    st.scale.copy_(torch.rand(st.scale.shape, generator=g, device=DEV))


def test_kv_copy_rows_exact_runs(gpu_lib):
    from opendecider_amd import kernels
    from opendecider_amd.kv_cache import StateKV
    src, dst = StateKV(3, 2, 4, 64, 300, DEV), StateKV(3, 1, 4, 64, 500, DEV)
    _rand_state(src, 1)
    dst.q.fill_(5)
    dst.scale.fill_(-2.0)
    segs = [(7 * i, 400 - 9 * i, 1 + (i * 5) % 9) for i in range(40)]          # 40 runs: two launches
    segs += [(0, 0, 0), (100, 420, 70)]                                        # an empty run, one of 70 rows
    sq, ss = src.state(1)
    dq, ds = dst.state(0)
    print("kv_copy_rows 42 runs", flush=True)
    kernels.kv_copy_rows(sq, ss, dq, ds, segs)
    torch.cuda.synchronize()
    want_q, want_s = torch.full_like(dq, 5), torch.full_like(ds, -2.0)
    for s0, d0, n in segs:                                                     # later runs win, as in the kernel
        want_q[:, :, d0:d0 + n] = sq[:, :, s0:s0 + n]
        want_s[:, :, d0:d0 + n] = ss[:, :, s0:s0 + n]
    assert torch.equal(dq, want_q) and torch.equal(ds.view(torch.int32), want_s.view(torch.int32))
    with pytest.raises(RuntimeError):                                          # past the destination: refused
        kernels.kv_copy_rows(sq, ss, dq, ds, [(0, 490, 20)])


def test_snapshot_restore_is_bit_exact(gpu_lib):
    from opendecider_amd.kv_cache import StateKV
    from opendecider_amd.state_cache import Int8PrefixCache
    L, H, D = 3, 4, 128
    st = StateKV(L, 1, H, D, 256, DEV)
    _rand_state(st, 2)
    st.set_length(200)
    store = Int8PrefixCache(L, H, D, 300, DEV)
    a = store.take(st, 0, "a", None, 120)
    b = store.take(st, 0, "b", a, 200)
    c = store.take(st, 0, "c", a, 150)                                         # a sibling branch off a
    for snap in (b, c, a):
        fresh = StateKV(L, 1, H, D, 256, DEV)
        fresh.q.fill_(9)
        print(f"restore {snap.key} ({snap.n_tokens} tokens)", flush=True)
        store.restore(snap, fresh, 0)
        torch.cuda.synchronize()
        n = snap.n_tokens
        assert fresh.length == n
        assert torch.equal(fresh.q[:, :, :, :n], st.q[:, :, :, :n])
        assert torch.equal(fresh.scale[:, :, :, :n].view(torch.int32), st.scale[:, :, :, :n].view(torch.int32))
        assert (fresh.q[:, :, :, n:] == 9).all()


def test_encode_resumes_from_the_deepest_prefix(gpu_lib):
    from opendecider_amd import decoder as dmod
    from opendecider_amd.state_cache import Int8PrefixCache
    cfg = dmod.DecoderConfig(n_layers=2, hidden=512, ffn=1024, n_heads=4, n_kv_heads=2, head_dim=128, vocab=1000)
    dec = dmod.random_decoder(cfg, seed=3, device=DEV, max_pos=2048)
    g = torch.Generator(device=DEV).manual_seed(4)
    A, B, C = (torch.randint(0, cfg.vocab, (n,), generator=g, device=DEV) for n in (300, 100, 60))
    store = Int8PrefixCache(cfg.n_layers, cfg.n_kv_heads, cfg.head_dim, 2048, DEV)
    s1 = dec.new_state_caches(1, 1024)
    print("encode [A, B]", flush=True)
    assert store.encode(dec, [A, B], s1) == 0 and s1.length == 400
    s2 = dec.new_state_caches(1, 1024)
    print("encode [A, B, C]", flush=True)
    assert store.encode(dec, [A, B, C], s2) == 400 and s2.length == 460       # [A, B] from the store
    ref = dec.new_state_caches(1, 1024)                                        # the same pieces, prefilled in order
    dec.prefill(torch.cat([A, B]).view(1, -1), ref)
    dec.prefill(C.view(1, -1), ref)
    torch.cuda.synchronize()
    n = 460
    assert torch.equal(s2.q[..., :n, :], ref.q[..., :n, :])
    assert torch.equal(s2.scale[..., :n].view(torch.int32), ref.scale[..., :n].view(torch.int32))
    assert store.encode(dec, [A, B, C], dec.new_state_caches(1, 1024)) == 460   # all of it cached now
    assert store.stats == {"hit_tokens": 860, "new_tokens": 460, "requests": 3}
