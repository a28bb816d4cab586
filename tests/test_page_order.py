"""The tests' conversion of K/V pools to the device page order, against that
order written out element by element: within a (block, layer) page of 16
tokens, per KV head of 64 dims (4 KB), key (slot, d) at float
(d/4)*64 + slot*4 + d%4 and value (slot, d) at (slot/4)*256 + d*4 + slot%4,
the order the fast and exact decode attention kernels read."""
import numpy as np

from .helpers import device_key_order, device_value_order


def test_device_page_order_element_by_element():
    blocks, layers, heads = 2, 2, 3
    pool = np.arange(blocks * layers * 16 * heads * 64, dtype=np.float32)
    k = device_key_order(pool, blocks, layers, heads)
    v = device_value_order(pool, blocks, layers, heads)
    assert k.size == v.size == pool.size
    for b in range(blocks):
        for l in range(layers):
            page = (b * layers + l) * 16 * heads * 64
            for slot in range(16):
                for h in range(heads):
                    for d in range(64):
                        want = pool[page + slot * heads * 64 + h * 64 + d]
                        base = page + h * 16 * 64
                        assert k[base + (d // 4) * 64 + slot * 4 + d % 4] == want
                        assert v[base + (slot // 4) * 256 + d * 4 + slot % 4] == want
