"""ggml tensor types on the hot path: ids and block geometry (crates/gguf/src/types.rs:74-122)."""


class GgmlType:
    F32 = 0
    F16 = 1
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    IQ2_XXS = 16
    IQ3_XXS = 18
    IQ2_S = 22
    IQ4_XS = 23
    BF16 = 30


# (elements per block, bytes per block)  types.rs:85-113
_BLOCK = {0: (1, 4), 1: (1, 2), 30: (1, 2), 8: (32, 34), 10: (256, 84), 11: (256, 110), 12: (256, 144),
          13: (256, 176), 14: (256, 210), 16: (256, 66), 18: (256, 98), 22: (256, 82), 23: (256, 136)}
TYPE_NAMES = {0: "F32", 1: "F16", 30: "BF16", 8: "Q8_0", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K",
              14: "Q6_K", 16: "IQ2_XXS", 18: "IQ3_XXS", 22: "IQ2_S", 23: "IQ4_XS"}


def block(ty):
    try:
        return _BLOCK[ty]
    except KeyError:
        raise ValueError(f"unsupported ggml type id {ty}") from None


def row_bytes(ty, n):
    """Bytes of a row of n elements; n must be a whole number of blocks (types.rs:118-122)."""
    be, bb = block(ty)
    if n % be:
        raise ValueError(f"{TYPE_NAMES[ty]}: row of {n} not a multiple of block {be}")
    return n // be * bb
