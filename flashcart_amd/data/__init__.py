from flashcart_amd.data.graph import AtomicGraph, batch_graphs, numbers_to_types, update_graph_positions
from flashcart_amd.data.neighbors import NeighborList, neighbor_pairs

__all__ = ["AtomicGraph", "batch_graphs", "numbers_to_types", "update_graph_positions", "NeighborList",
           "neighbor_pairs"]
