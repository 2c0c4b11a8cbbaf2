from isa.operators.cim import CIMLinear, HybridFFN, PhysicalFFN, VoltageMapping

__all__ = ["CIMLinear", "HybridFFN", "PhysicalFFN", "VoltageMapping"]
