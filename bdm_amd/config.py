"""Bank geometry for the BDM routed-memory layer.

The field names, defaults and validation rules follow the reference
configuration (``implementation/bdm/config.py:16-84`` and
``implementation/bsdm/__init__.py:10-15``) so that a configuration record
written by the reference loads here unchanged.
"""

from __future__ import annotations

import math
from dataclasses import asdict, dataclass


def near_square_factors(value: int) -> tuple[int, int]:
    """Split ``value`` into ``(a, b)`` with ``a * b == value`` and ``a`` the
    largest divisor not above ``sqrt(value)`` (``config.py:7-13``)."""
    if value <= 0:
        raise ValueError('value must be positive')
    first = math.isqrt(value)
    while value % first:
        first -= 1
    return first, value // first


def replay_interval(bank_size: int) -> int:
    """Events between BF16 state roundings on the training path.

    ``min(16, max(4, 128 // next_pow2(S)))`` (``role_bank_kernel.py:153-154``,
    ``model.py:131``): 16 for S <= 8, 8 for S = 16, 4 for S >= 32.
    """
    pow2 = 1 << (bank_size - 1).bit_length()
    return min(16, max(4, 128 // pow2))


@dataclass(frozen=True)
class BDMConfig:
    dim: int = 128
    bank_count: int = 1024
    bank_size: int = 4
    selected_banks: int = 8
    value_width: int = 128
    norm_eps: float = 1e-5
    num_heads: int = 1
    routed_decay: bool = False
    qk_normalization: str = 'original'
    output_normalization: str = 'rms'
    output_bias: bool = False
    training_state_dtype: str = 'bfloat16'

    def __post_init__(self):
        # The same conditions as the reference config (config.py:31-51), so a
        # geometry accepted there is accepted here and vice versa.
        sizes = ('dim', 'bank_count', 'bank_size', 'selected_banks', 'value_width', 'num_heads')
        bad = [name for name in sizes if type(getattr(self, name)) is not int or getattr(self, name) < 1]
        if bad:
            raise ValueError(f'BDM config: {", ".join(bad)} needs a positive int')
        checks = (
            (self.bank_size <= 256, f'BDM config: bank_size {self.bank_size} exceeds the 256-row limit'),
            (self.value_width % self.num_heads == 0,
             f'BDM config: {self.num_heads} heads do not split value_width {self.value_width} evenly'),
            (type(self.routed_decay) is bool and type(self.output_bias) is bool,
             'BDM config: routed_decay and output_bias take True or False'),
            (self.qk_normalization in ('original', 'nvidia'),
             f'BDM config: qk_normalization {self.qk_normalization!r} is neither original nor nvidia'),
            (self.output_normalization in ('rms', 'layer'),
             f'BDM config: output_normalization {self.output_normalization!r} is neither rms nor layer'),
            (self.training_state_dtype in ('float32', 'bfloat16'),
             f'BDM config: training_state_dtype {self.training_state_dtype!r} is neither float32 nor bfloat16'),
            (self.selected_banks <= min(near_square_factors(self.bank_count)),
             f'BDM config: the product-key router picks {self.selected_banks} banks, more than the smaller '
             f'factor of {self.bank_count} holds'),
            (math.isfinite(self.norm_eps) and self.norm_eps > 0,
             f'BDM config: norm_eps {self.norm_eps} is not a finite positive number'),
        )
        for ok, message in checks:
            if not ok:
                raise ValueError(message)

    @property
    def logical_rows(self) -> int:
        return self.bank_count * self.num_heads * self.bank_size

    @property
    def reads(self) -> int:
        return self.selected_banks * self.num_heads * self.bank_size

    @property
    def writes(self) -> int:
        return self.reads

    @property
    def head_value_width(self) -> int:
        return self.value_width // self.num_heads

    @property
    def route_factors(self) -> tuple[int, int]:
        return near_square_factors(self.bank_count)

    @property
    def initial_factors(self) -> tuple[int, int]:
        return near_square_factors(self.logical_rows)

    def record(self) -> dict:
        return dict(asdict(self), logical_rows=self.logical_rows, R=self.reads, W=self.writes,
                    read_banks=self.selected_banks, write_banks=self.selected_banks,
                    router='shared_residual_product_key', memory_rule='gdn2')

    @classmethod
    def from_record(cls, record: dict) -> 'BDMConfig':
        # Records older than a field leave it out; they load as one head, an
        # FP32 training state and the class defaults for the other options.
        optional = ('routed_decay', 'qk_normalization', 'output_normalization', 'output_bias')
        filled = {'num_heads': 1, 'training_state_dtype': 'float32',
                  **{name: cls.__dataclass_fields__[name].default for name in optional}, **record}
        config = cls(**{name: filled[name] for name in cls.__dataclass_fields__})
        if filled != config.record():
            raise ValueError('BDM record: its derived fields (rows, reads, writes, router, rule) do not match '
                             'the configuration they were stored with')
        return config


@dataclass(frozen=True)
class BSDMConfig(BDMConfig):
    """Block-sparse delta memory defaults (``bsdm/__init__.py:10-15``)."""
    routed_decay: bool = True
    qk_normalization: str = 'nvidia'
    output_normalization: str = 'layer'
    output_bias: bool = True
