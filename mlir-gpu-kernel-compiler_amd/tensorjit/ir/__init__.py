from .graph import OPS, DType, Graph, Node, OpKind, TensorType, broadcast_shapes, infer_type
from .printer import print_graph

__all__ = ["OPS", "DType", "Graph", "Node", "OpKind", "TensorType", "broadcast_shapes", "infer_type", "print_graph"]
