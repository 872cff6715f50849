from ssd.models.bridges import TransitionBridge
from ssd.models.llama import LlamaShape, MI355XLlama
from ssd.models.subnetwork_draft import BridgeSpec, DraftOutput, SubnetworkDraftModel, plan_bridges

__all__ = ["BridgeSpec", "DraftOutput", "LlamaShape", "MI355XLlama", "SubnetworkDraftModel", "TransitionBridge",
           "plan_bridges"]
