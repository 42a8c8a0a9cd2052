"""Cache-argument checks of the block chain, on the CPU (no kernel is reached): a write slot
that is also read, cached tables that disagree with the slot's length, empty slots, rotated
slots given tables, and write lengths that do not fit."""
import pytest
import torch

from joyomni_ops.dit_block import CachedChunk, KVRing, QuantizedDoubleStreamBlock

check = QuantizedDoubleStreamBlock.check_cache_args


def _ring():
    r = KVRing(4, 32, 2, 128, "cpu")
    r.lengths = [16, 32, 0, 8]
    return r


def _tables(n):
    return torch.ones(n, 128), torch.zeros(n, 128)


def test_valid_arguments_pass():
    r = _ring()
    check(24, r, 2, [CachedChunk(0, *_tables(16)), CachedChunk(1, *_tables(32))], 24)
    check(24, r, None, [CachedChunk(3, *_tables(8))], 24)
    check(24, None, None, [], 24)
    r.pre_rope[3] = False
    check(24, r, 2, [CachedChunk(3)], 10)


def test_write_slot_that_is_also_read_is_rejected():
    r = _ring()
    with pytest.raises(ValueError, match="write_slot 0 is also a cached slot"):
        check(24, r, 0, [CachedChunk(0, *_tables(16))], 24)


def test_table_rows_must_match_slot_length():
    r = _ring()
    with pytest.raises(ValueError, match="holds 16 tokens but its cos table"):
        check(24, r, 2, [CachedChunk(0, *_tables(15))], 24)
    c, s = _tables(16)
    with pytest.raises(ValueError, match="its sin table"):
        check(24, r, 2, [CachedChunk(0, c, s[:8])], 24)


def test_empty_missing_and_repeated_slots_are_rejected():
    r = _ring()
    with pytest.raises(ValueError, match="cached slot 2 is empty"):
        check(24, r, 1, [CachedChunk(2, *_tables(0))], 24)
    with pytest.raises(ValueError, match="needs its cos/sin tables"):
        check(24, r, 2, [CachedChunk(0)], 24)
    with pytest.raises(ValueError, match="attended twice"):
        check(24, r, 2, [CachedChunk(0, *_tables(16)), CachedChunk(0, *_tables(16))], 24)
    with pytest.raises(ValueError, match="not a slot"):
        check(24, r, 2, [CachedChunk(7, *_tables(16))], 24)
    r.pre_rope[3] = False
    with pytest.raises(ValueError, match="holds rotated K; it takes no RoPE tables"):
        check(24, r, 2, [CachedChunk(3, *_tables(8))], 24)


def test_write_bounds():
    r = _ring()
    with pytest.raises(ValueError, match="not a slot of the ring"):
        check(24, r, 4, [], 24)
    with pytest.raises(ValueError, match="outside"):
        check(24, r, 1, [], 25)
    with pytest.raises(ValueError, match="do not fit"):
        check(40, r, 1, [], 40)
    with pytest.raises(ValueError, match="need a KV ring"):
        check(24, None, 1, [], 24)


def test_adjacent_cached_tables_are_joined_without_a_copy():
    """Two chunks' tables cut from one table of every cached token are joined as a view; any other
    pair (reversed, separate buffers) is copied, and both give the rows of a then b."""
    from joyomni_ops.dit_block import _adjacent_rows
    full = torch.arange(12 * 4, dtype=torch.float32).reshape(12, 4)
    a, b = full[:5], full[5:]
    v = _adjacent_rows(a, b)
    assert v.data_ptr() == full.data_ptr() and torch.equal(v, full)
    r = _adjacent_rows(b, a)
    assert r.data_ptr() != full.data_ptr() and torch.equal(r, torch.cat([b, a]))
    c = _adjacent_rows(a.clone(), b.clone())
    assert torch.equal(c, full)
    gap = _adjacent_rows(full[:4], full[5:])
    assert torch.equal(gap, torch.cat([full[:4], full[5:]]))


def test_cached_rows_stamp_tracks_every_input_of_the_assembly():
    """JointKV reuses the assembled cached rows only while this stamp is unchanged: it must move
    with a write to a cached slot (through torch or through the block), the slot's length or
    storage mode, a different or modified table, and a different ring; and stay put otherwise."""
    from joyomni_ops.dit_block import cached_rows_stamp
    r = _ring()
    c0, s0 = _tables(16)
    c1, s1 = _tables(32)
    cached = [CachedChunk(0, c0, s0), CachedChunk(1, c1, s1)]
    base = cached_rows_stamp(r, cached)
    assert cached_rows_stamp(r, cached) == base
    assert cached_rows_stamp(r, []) == ()
    r.touch(2)                                   # a slot that is not read
    assert cached_rows_stamp(r, cached) == base
    changes = []
    r.k[1, 0].add_(1.0)                          # in-place write through a view of the ring
    changes.append(cached_rows_stamp(r, cached))
    r.v[0, 3].mul_(2.0)
    changes.append(cached_rows_stamp(r, cached))
    r.touch(1)                                   # a kernel rewrote a read slot
    changes.append(cached_rows_stamp(r, cached))
    r.lengths[0] = 15
    changes.append(cached_rows_stamp(r, [CachedChunk(0, *_tables(15)), cached[1]]))
    r.lengths[0] = 16
    r.pre_rope[1] = False
    changes.append(cached_rows_stamp(r, cached))
    r.pre_rope[1] = True
    c1.add_(0.5)                                 # a table modified in place
    changes.append(cached_rows_stamp(r, cached))
    changes.append(cached_rows_stamp(r, [cached[0], CachedChunk(1, c1.clone(), s1)]))  # another tensor
    changes.append(cached_rows_stamp(_ring(), cached))                                   # another ring
    seen = [base]
    for st in changes:
        assert st not in seen, st
        seen.append(st)


def test_cached_rows_stamp_holds_its_tables_and_tells_a_rebuilt_table_at_the_same_address():
    """A table built per forward and dropped on return may have its address handed to the next
    forward's table. The stamp keeps every table it names alive (so the address cannot be
    recycled while the stamp exists) and compares them by identity: a different tensor with the
    same address, shape, strides, dtype and version counter but other contents does not match."""
    import gc
    import weakref

    from joyomni_ops.dit_block import cached_rows_stamp
    r = _ring()
    cos, sin = _tables(16)
    ref = weakref.ref(cos)
    # a tensor aliasing the same memory with the same data_ptr, shape, strides, dtype and version
    # counter (set_ leaves the alias at version 1; one in-place no-op puts the table there too)
    alias = torch.empty(0).set_(cos.untyped_storage(), cos.storage_offset(), cos.shape, cos.stride())
    cos.mul_(1.0)
    assert alias.data_ptr() == cos.data_ptr() and alias._version == cos._version == 1
    stamp = cached_rows_stamp(r, [CachedChunk(0, cos, sin)])
    alias.numpy()[:] = 0.25                      # a raw write that no version counter sees
    assert cached_rows_stamp(r, [CachedChunk(0, alias, sin)]) != stamp
    assert cached_rows_stamp(r, [CachedChunk(0, cos, sin)]) == stamp
    del cos, alias
    gc.collect()
    assert ref() is not None                     # the stamp keeps the table (and its address) alive
    del stamp
    gc.collect()
    assert ref() is None
    # a ring rebuilt from scratch (generations reset to 0) is another ring
    r2 = _ring()
    c2, s2 = _tables(16)
    assert cached_rows_stamp(r2, [CachedChunk(0, c2, s2)]) != cached_rows_stamp(r, [CachedChunk(0, c2, s2)])
