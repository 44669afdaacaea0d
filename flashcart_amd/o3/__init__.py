"""Cartesian tensor expansions, tensor products and equivariant linear maps on MI355X."""

from flashcart_amd.o3.irreps import Irreps
from flashcart_amd.o3.tensor_product import TensorProduct
from flashcart_amd.o3.linear import LinearLayer
from flashcart_amd.o3 import utils
from flashcart_amd.o3._graph import GraphCSR, build_graph

__all__ = ["Irreps", "TensorProduct", "LinearLayer", "utils", "GraphCSR", "build_graph"]
