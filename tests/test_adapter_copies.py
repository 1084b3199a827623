"""The fp16 adapter-copy cache (`adapters.AdapterCopies`) on the CPU: a copy made outside the
flat layout is served again only for the very weight it was made from.

A training process that rebuilds its model can get a new adapter weight with the id, storage
address and version counter of a freed one. q and v adapters of one width share a shape, so this
happens readily. A cache keyed on those alone would then hand the new weight the old weight's
copy. That is what a sequence of GPU tests building one model per case ran into. Here the reuse
is forced by planting the entry, since the allocator's addresses cannot be steered. (Only a
weight's first copy is made on the CPU path; later ones refresh the flat layout on the GPU.)
"""

import weakref

import torch

from talm_amd.adapters import AdapterCopies, _key


def test_a_copy_is_served_only_for_the_weight_it_was_made_from():
    copies = AdapterCopies()
    old = torch.full((16, 8), 3.0)
    new = torch.full((16, 8), -1.0)
    assert torch.equal(copies.half(old), old.half())
    # the entry that a freed weight would leave under the new weight's id, with the new weight's
    # key (same storage address and version)
    copies.loose[id(new)] = (weakref.ref(old), _key(new), old.half())
    assert torch.equal(copies.half(new), new.half())
    # the same for the transposed side-by-side copies of a q|k|v node's two adapters
    a_q, a_v = torch.randn(16, 8), torch.randn(16, 8)
    stale = torch.randn(8, 32).half()
    copies.loose[(id(a_q), id(a_v))] = ((weakref.ref(old), weakref.ref(new)),
                                       (_key(a_q), _key(a_v)), stale)
    want = torch.cat([a_q, a_v], 0).t().half()
    assert torch.equal(copies.pair_t([a_q, a_v]), want)
