from .graph import Graph, Node, Value
from .types import Buffer, Layout, contiguous_strides

__all__ = ["Buffer", "Layout", "contiguous_strides", "Graph", "Node", "Value"]
