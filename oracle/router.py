"""Router closed form (reference src/dynakv/kernels/router.py:14-17). Test infrastructure only."""


def select(cache_length: int, switch_tokens: int = 500) -> str:
    # router.py:15-16: negative lengths are rejected
    if cache_length < 0:
        raise ValueError("cache_length must be non-negative")
    # router.py:17: strict comparison, post-append length
    return "short_fused" if cache_length < switch_tokens else "long_two_stage"
