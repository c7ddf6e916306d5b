"""MI355X-native routed-memory path of the Block Delta Memory layer.

Public surface mirrors the reference packages ``bdm`` and ``bsdm``:
``BDMConfig``/``BSDMConfig``, the ``BankedDeltaMemory`` module (alias
``BlockSparseDeltaMemory``), the routed operator ``bank_training``, the
router ``product_key_route``, ``bank_occupancy`` (the bank-union
regularizer), ``written_banks`` (the copy-on-write state count at nested
prefixes) and ``GraphDecoder`` (a layer's decode step replayed from a HIP
graph).  Kernels live in ``libbdm_hip.so``.
"""

from .config import BDMConfig, BSDMConfig, near_square_factors, replay_interval
from .graphs import GraphDecoder, LanguageModelGraphDecoder
from .model import BankedDeltaMemory
from .ops import route_validation, set_route_validation
from .occupancy import bank_occupancy, written_banks
from .routed_update import bank_training, role_bank_training
from .routing import SharedResidualRouter, product_key_route

BlockSparseDeltaMemory = BankedDeltaMemory

__all__ = ['BDMConfig', 'BSDMConfig', 'BankedDeltaMemory', 'BlockSparseDeltaMemory', 'GraphDecoder',
           'LanguageModelGraphDecoder',
           'SharedResidualRouter', 'bank_occupancy', 'bank_training', 'role_bank_training', 'product_key_route',
           'near_square_factors', 'replay_interval', 'route_validation', 'set_route_validation', 'written_banks']
