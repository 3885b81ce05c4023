"""Host logic of the preallocated KV-cache store (transformer_amd/latent_cache.py), on CPU
tensors: appends match the reference's torch.cat growth (transformer.py:215-218,241-244),
a dict a caller holds never changes under it, capacity grows geometrically."""
import pytest
import torch

from transformer_amd import latent_cache as LC


def _cat_reference(cache, lat, kr):
    if cache is None:
        return lat.clone(), kr.clone()
    return torch.cat([cache["latent"], lat], 1), torch.cat([cache["k_rope"], kr], 2)


def _rand(B, T, DL=16, Hr=1, dr=8, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, T, DL, generator=g), torch.randn(B, Hr, T, dr, generator=g)


def test_grown_capacity():
    assert LC.grown_capacity(0, 1000) == 256
    assert LC.grown_capacity(100, 1000) == 256
    assert LC.grown_capacity(300, 1000) == 512
    assert LC.grown_capacity(900, 1000) == 1000  # capped at the limit
    assert LC.grown_capacity(1000, 1000) == 1000
    for need in range(0, 5000, 37):
        c = LC.grown_capacity(need, 1 << 20)
        assert c >= need and c % 256 == 0 and c >= need * 3 // 2


def test_appends_match_cat_and_stay_in_place():
    with torch.no_grad():
        cache, ref = None, None
        stores = set()
        for step, T in enumerate([5, 1, 1, 3, 1, 40]):
            lat, kr = _rand(2, T, seed=step)
            a, b, cache = LC.append(cache, lat, kr, max_len=4096)
            ref = _cat_reference(ref and {"latent": ref[0], "k_rope": ref[1]}, lat, kr)
            assert torch.equal(a, ref[0]) and torch.equal(b, ref[1])
            assert torch.equal(cache["latent"], ref[0]) and torch.equal(cache["k_rope"], ref[1])
            assert cache["seq_len"] == ref[0].size(1)
            assert tuple(cache["latent"].shape) == tuple(ref[0].shape)
            assert tuple(cache["k_rope"].shape) == tuple(ref[1].shape)
            stores.add(id(LC.store_of(cache)))
        assert len(stores) == 1  # 51 tokens fit the first 256-token buffers: never copied


def test_branching_from_an_older_dict_copies():
    with torch.no_grad():
        lat0, kr0 = _rand(1, 10, seed=1)
        _, _, c0 = LC.append(None, lat0, kr0, max_len=4096)
        lat1, kr1 = _rand(1, 1, seed=2)
        _, _, c1 = LC.append(c0, lat1, kr1, max_len=4096)
        saved = c1["latent"].clone(), c1["k_rope"].clone()
        # c0 is no longer the newest dict of its buffers: branching from it must not touch c1
        assert LC.store_of(c0) is None
        lat2, kr2 = _rand(1, 1, seed=3)
        _, _, c2 = LC.append(c0, lat2, kr2, max_len=4096)
        assert torch.equal(c1["latent"], saved[0]) and torch.equal(c1["k_rope"], saved[1])
        assert torch.equal(c2["latent"], torch.cat([lat0, lat2], 1))
        assert torch.equal(c2["k_rope"], torch.cat([kr0, kr2], 2))
        assert LC.store_of(c2) is not LC.store_of(c1)
        # the old prefix is still intact
        assert torch.equal(c0["latent"], lat0) and torch.equal(c0["k_rope"], kr0)


def test_growth_past_capacity_and_foreign_cache():
    with torch.no_grad():
        lat, kr = _rand(2, 300, seed=4)
        foreign = {"latent": lat, "k_rope": kr, "seq_len": 300}  # a cache made elsewhere
        lat1, kr1 = _rand(2, 10, seed=5)
        _, _, c = LC.append(foreign, lat1, kr1, max_len=4096)
        s = LC.store_of(c)
        assert s is not None and s.capacity == 512 and c["seq_len"] == 310
        lat2, kr2 = _rand(2, 300, seed=6)
        _, _, c2 = LC.append(c, lat2, kr2, max_len=4096)  # 610 > 512: regrow
        s2 = LC.store_of(c2)
        assert s2 is not s and s2.capacity >= 610
        assert torch.equal(c2["latent"], torch.cat([lat, lat1, lat2], 1))
        assert torch.equal(c2["k_rope"], torch.cat([kr, kr1, kr2], 2))


def test_dtype_change_and_limits():
    with torch.no_grad():
        lat, kr = _rand(1, 4, seed=7)
        _, _, c = LC.append(None, lat, kr, max_len=8)
        lat16, kr16 = lat.bfloat16(), kr.bfloat16()
        _, _, c16 = LC.append(c, lat16, kr16, max_len=8)  # new dtype: fresh bf16 buffers
        assert c16["latent"].dtype == torch.bfloat16 and c16["seq_len"] == 8
        assert torch.equal(c16["latent"][:, :4], lat.bfloat16())
        with pytest.raises(ValueError):
            LC.append(c16, lat16[:, :1], kr16[:, :, :1], max_len=8)
    with pytest.raises(RuntimeError):
        LC.append(None, lat, kr, max_len=8)  # autograd on
