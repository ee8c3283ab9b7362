"""KV budget helpers (device.h:36-50, 148-190): the exact byte counts the
reference's check_kvtype.hip:132-174 pins at 131072 tokens, the general-shape
form, and the largest context that fits a budget (288 GB MI355X HBM)."""
import pytest

# check_kvtype.hip:150-159: (K, V) -> bytes at 131072 tokens
GOLDEN_131K = {
    ("f16", "f16"): 8589934592,
    ("q8_0", "q8_0"): 4563402752,
    ("q4_0", "q4_0"): 2415919104,
    ("q5_0", "q4_1"): 2818572288,
    ("q8_0", "q4_0"): 3489660928,
    ("q5_0", "q4_0"): 2684354560,
    ("q8_0", "q4_1"): 3623878656,
}


@pytest.mark.parametrize("pair", sorted(GOLDEN_131K))
def test_kv_cache_bytes_reference_values(rd4, pair):
    kt, vt = (rd4.kv_type_parse(x) for x in pair)
    assert rd4.kv_cache_bytes(131072, kt, vt) == GOLDEN_131K[pair]
    # the same through the general shape (16 layers x 4 kv heads x 256 dims)
    assert rd4.kv_cache_bytes(131072, kt, vt, 16, 4, 256) == GOLDEN_131K[pair]


def test_kv_cache_bytes_per_token_closed_form(rd4):
    # row bytes x heads x layers per side, exact for every type at head_dim 256
    for kt in range(6):
        for vt in range(6):
            per_tok = 16 * 4 * (rd4.kv_row_bytes(kt, 256) + rd4.kv_row_bytes(vt, 256))
            assert rd4.kv_cache_bytes(1000, kt, vt) == 1000 * per_tok
    assert rd4.kv_cache_bytes(10, 99, 1) == 0
    assert rd4.kv_cache_bytes(10, 1, 1, 0, 4, 256) == 0


@pytest.mark.parametrize("kt,vt", [(1, 1), (2, 2), (3, 3), (4, 5), (2, 3)])
def test_kv_max_ctx_is_the_largest_that_fits(rd4, kt, vt):
    budget, reserved = 288 * 10**9, 60 * 10**9  # 288 GB HBM, ~60 GB of weights and buffers
    c = rd4.kv_max_ctx(budget, reserved, 64, 8, 128, kt, vt)
    avail = budget - reserved
    assert 0 < c < (1 << 24)
    assert rd4.kv_cache_bytes(c, kt, vt, 64, 8, 128) <= avail
    assert rd4.kv_cache_bytes(c + 1, kt, vt, 64, 8, 128) > avail


def test_kv_max_ctx_caps_and_rejects(rd4):
    # reference shape at q4_0 in 288 GB with 20 GB reserved: 18432 B/token
    assert rd4.kv_max_ctx(288 * 10**9, 20 * 10**9, 16, 4, 256, 3, 3) == 268 * 10**9 // 18432
    assert rd4.kv_max_ctx(10**12, 0, 16, 4, 256, 3, 3) == 1 << 24   # capped at kMaxCtxSize
    assert rd4.kv_max_ctx(10, 20, 16, 4, 256, 1, 1) == 0       # reserved > budget
    assert rd4.kv_max_ctx(10**12, 0, 16, 4, 256, 7, 1) == 0    # bad type
