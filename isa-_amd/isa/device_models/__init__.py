from isa.device_models.config import (
    FLASH_TRANSISTOR_EKV_CONFIG,
    FLASH_TRANSISTOR_PARAMETERS,
    make_flash_transistor_ekv_config,
)

__all__ = [
    "FLASH_TRANSISTOR_EKV_CONFIG",
    "FLASH_TRANSISTOR_PARAMETERS",
    "make_flash_transistor_ekv_config",
]
